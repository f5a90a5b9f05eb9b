// C-ABI of libcqhip (include/cqhip.h): the host side of go-whistle's
// internal/cq Matrix API and the int8 KV entry points, over the gfx950
// kernels of cq_kernels.hip and int8_kernels.hip.
//
// A cq_matrix is a view {storage, first row, rows, exact} of an immutable
// device storage shared by every view (internal/cq/matrix.go:25-41, 131-157).
// Validation, error texts and the Bytes accounting follow the reference
// (matrix.go:46-145, kernel.go:100-158); shape misuse, which the Go API
// answers with a panic, returns CQ_ERR_MISUSE with the panic's text.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/cqhip.h"
#include "cq_internal.hpp"

using namespace cqhip;

namespace {

thread_local std::string t_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    t_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(CQ_ERR_DEVICE, "cq: %s: %s", what, hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                          \
    do {                                             \
        hipError_t e_ = (expr);                      \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

struct DeviceInfo {
    int device = -1;
    int cus = 256;
    size_t max_lds = 64 * 1024;
    std::string name;
};

DeviceInfo &device_info() {
    static DeviceInfo info;
    static std::once_flag once;
    std::call_once(once, [] {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) != hipSuccess) return;
        info.device = dev;
        info.cus = p.multiProcessorCount;
        info.max_lds = std::max<size_t>(p.sharedMemPerBlock, 64 * 1024);
        info.name = p.gcnArchName;
    });
    return info;
}

// Per-thread stream and device staging for the host-slice calls.
struct Staging {
    hipStream_t stream = nullptr;
    void *buf = nullptr;
    size_t cap = 0;
    ~Staging() {
        if (buf) (void)hipFree(buf);
        if (stream) (void)hipStreamDestroy(stream);
    }
    hipError_t ensure(size_t bytes) {
        if (!stream) {
            hipError_t e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
            if (e != hipSuccess) return e;
        }
        if (bytes <= cap) return hipSuccess;
        if (buf) (void)hipFree(buf);
        buf = nullptr;
        cap = 0;
        size_t want = std::max<size_t>(bytes, 1 << 20);
        hipError_t e = hipMalloc(&buf, want);
        if (e != hipSuccess) return e;
        cap = want;
        return hipSuccess;
    }
};
thread_local Staging t_stage;

size_t align256(size_t n) { return (n + 255) & ~static_cast<size_t>(255); }

}  // namespace

// ---- matrix storage and views -----------------------------------------------

struct CqStore {
    int out, in, group, groups, width, row_bytes, group_bytes, unit_bytes, units, nblk;
    float cb[16];
    int ncb;
    float cb_max, lut_step, inv_sqrt;
    uint8_t *d_idx = nullptr;
    uint16_t *d_norm = nullptr;
    size_t idx_bytes = 0, norm_bytes = 0;
    std::atomic<bool> prepared{false};
    ~CqStore() {
        if (d_idx) (void)hipFree(d_idx);
        if (d_norm) (void)hipFree(d_norm);
    }
};

struct cq_matrix {
    std::shared_ptr<CqStore> st;
    int row0, out;
    bool exact;
    bool dense = false;  // a Dense view: Exact's semantics, batched products on the fp32 MFMA form
};

namespace {

// best() (internal/cq/kernel.go:92-98): lut unless Exact or the groups are
// wider than the lut kernel's 256 bytes.
bool uses_lut(const cq_matrix *m) { return !m->exact && m->st->group_bytes <= kLutMaxGroupBytes; }

float gomax(float a, float b) {
    if (a != a || b != b) return NAN;
    return a > b ? a : b;
}

// The shared-table test of lut.go:206-209.
bool shares_tables(const CqStore &a, const CqStore &b) {
    if (a.in != b.in || a.group != b.group || a.width != b.width || a.cb_max != b.cb_max) return false;
    for (int c = 0; c < a.ncb; ++c)
        if (a.cb[c] != b.cb[c]) return false;
    return true;
}

struct LaunchPlan {
    int tb, gc;
    size_t lds;
};

LaunchPlan plan(const CqStore &s, int mode, long long nblk_total, int rows) {
    const DeviceInfo &d = device_info();
    LaunchPlan p;
    // Up to four blocks per tile once there are enough tiles to fill the chip.
    long long want = 2LL * d.cus;
    long long work = nblk_total * std::max(rows, 1);
    p.tb = static_cast<int>(std::min<long long>(4, std::max<long long>(1, work / want)));
    const size_t budget = std::min<size_t>(d.max_lds, 96 * 1024);
    p.gc = s.groups;
    while (p.gc > 1 && product_lds_bytes(s.width, s.group_bytes, mode, p.gc, p.tb) > budget) p.gc--;
    p.lds = product_lds_bytes(s.width, s.group_bytes, mode, p.gc, p.tb);
    return p;
}

int check_geometry(const CqStore &s, int mode) {
    if (mode == kModeLut && s.group_bytes > kLutMaxGroupBytes)
        return fail(CQ_ERR_UNSUPPORTED, "cq: lut kernel with %d index bytes per group", s.group_bytes);
    if (s.group_bytes > 512)
        return fail(CQ_ERR_UNSUPPORTED, "cq: group %d of %d bits is wider than this library runs", s.group, s.width);
    const size_t need = product_lds_bytes(s.width, s.group_bytes, mode, 1, 1);
    if (need > device_info().max_lds)
        return fail(CQ_ERR_UNSUPPORTED, "cq: group %d needs %zu bytes of LDS", s.group, need);
    return CQ_OK;
}

void fill_common(ProdArgs &a, const CqStore &s, int rows) {
    a.in = s.in;
    a.groups = s.groups;
    a.row_bytes = s.row_bytes;
    a.rows = rows;
    for (int c = 0; c < 16; ++c) a.cb[c] = c < s.ncb ? s.cb[c] : 0.0f;
    a.cb_max = s.cb_max;
    a.lut_step = s.lut_step;
    a.inv_sqrt = s.inv_sqrt;
    a.nib4_rows = rows - rows % 4;  // gemmScalar (kernel.go:170-183)
}

void fill_job(JobDesc &j, const cq_matrix *m, const float *x, float *y, int rows) {
    const CqStore &s = *m->st;
    std::memset(&j, 0, sizeof j);
    j.idx = s.d_idx;
    j.norm = s.d_norm;
    j.x = x;
    j.y = y;
    j.x_stride = s.in;
    j.y_stride = m->out;
    j.row0 = m->row0;
    j.out = m->out;
    j.blk0 = m->row0 / kBlockRows;
    j.nblk = (m->row0 + m->out + kBlockRows - 1) / kBlockRows - j.blk0;
    j.in = s.in;
    j.groups = s.groups;
    j.units = s.units;
    j.rows = rows;
    for (int c = 0; c < 16; ++c) j.cb[c] = c < s.ncb ? s.cb[c] : 0.0f;
    j.cb_max = s.cb_max;
    j.lut_step = s.lut_step;
}

// A fused prologue/epilogue request (see JobDesc).
struct Fuse {
    const float *ngain = nullptr;
    const float *resid = nullptr;
    long long resid_stride = 0;
    int act = 0;
    const float *xgate = nullptr;  // the product is of x * sigmoid(xgate)
    // int8 appends of matrix k of the call (null arrays / entries: none)
    int8_t *const *app_q = nullptr;
    float *const *app_s = nullptr;
    const float *const *app_cos = nullptr;
    const float *const *app_sin = nullptr;
    long long app_q_stride = 0, app_s_stride = 0;
    const int32_t *app_pos = nullptr;
    int app_cap = 0;
    bool any() const { return ngain || resid || act || xgate || app_q; }
};

// Job j runs matrix k of the call.
void apply_fuse(JobDesc &j, const Fuse *f, int k) {
    if (!f) return;
    j.ngain = f->ngain;
    j.resid = f->resid;
    j.resid_stride = f->resid_stride;
    j.act = f->act;
    j.xgate = f->xgate;
    if (f->app_q && f->app_q[k]) {
        j.app_q = f->app_q[k];
        j.app_s = f->app_s[k];
        j.app_q_stride = f->app_q_stride;
        j.app_s_stride = f->app_s_stride;
        j.app_pos = f->app_pos;
        j.app_cap = f->app_cap;
        if (f->app_cos && f->app_cos[k]) {
            j.app_cos = f->app_cos[k];
            j.app_sin = f->app_sin[k];
        }
    }
}

constexpr int kLutTile = 4;     // blocks per tile of the lut kernel
constexpr int kLutChunk = 4;    // groups per LDS chunk
constexpr int kLutMaxBpw = 16;  // most blocks per workgroup
// LDS a chunk may take when a launch widens its chunks (six workgroups of the
// 2-bit kernel per CU; wider chunks lost: 16 groups of 512x2048 CQ2 at 256
// activations 25.5 us, 8 groups of 512x2048 CQ4 36.5 us against 29.7 with 4)
constexpr size_t kLutChunkLds = 26 * 1024;

int lut_chunk(int groups_max) { return std::min(kLutChunk, std::max(1, groups_max)); }

// The lut kernel runs a geometry whose chunk of tables fits in LDS.
bool lut_fits(const CqStore &s) {
    return lut_geometry_supported(s.width, s.group_bytes) &&
           lut_lds_bytes(s.width, s.group_bytes, lut_chunk(s.groups), kLutTile, kLutMaxBpw) <=
               std::min<size_t>(device_info().max_lds, 128 * 1024);
}

// The same number of units of at most b blocks each, as even as possible:
// 8 blocks at 6 per unit become 4 + 4, not 6 + 2 (a short unit still pays
// a full build of its activation's tables).
int balanced_blocks(int nblk, int b) {
    const int units = (nblk + b - 1) / b;
    return std::max(1, (nblk + units - 1) / units);
}

int blocks_per_workgroup(long long blocks) {
    const long long want = 4LL * device_info().cus;
    return static_cast<int>(std::min<long long>(kLutMaxBpw, std::max<long long>(1, blocks / want)));
}

// One launch of the lut kernel for up to kKernargJobs views of one geometry
// and the same activations.
int run_lut(cq_matrix *const *ms, int n, float *const *dsts, const float *x, int rows, hipStream_t stream,
            const Fuse *fz = nullptr, const TabOut *to = nullptr, int *built = nullptr) {
    const CqStore &s0 = *ms[0]->st;
    LutLaunch a;
    std::memset(&a, 0, sizeof a);
    long long blocks = 0;
    int groups_max = 0;
    for (int k = 0; k < n; ++k) {
        if (ms[k]->out == 0) continue;
        JobDesc &j = a.jobs[a.njobs++];
        fill_job(j, ms[k], x, dsts[k], rows);
        apply_fuse(j, fz, k);
        blocks += static_cast<long long>(j.nblk) * rows;
        groups_max = std::max(groups_max, j.groups);
    }
    if (a.njobs == 0 || rows == 0) return CQ_OK;
    int nmax = 0;
    for (int k = 0; k < a.njobs; ++k) nmax = std::max(nmax, a.jobs[k].nblk);
    a.bpw = balanced_blocks(nmax, blocks_per_workgroup(blocks));
    const int wg = (nmax + a.bpw - 1) / a.bpw;  // grid x: the units of the largest job (grid z: the jobs)
    long long units = 0;
    for (int k = 0; k < a.njobs; ++k) units += (a.jobs[k].nblk + a.bpw - 1) / a.bpw;
    a.tb = kLutTile;
    a.gc = lut_chunk(groups_max);
    // Wider rows take their tables in fewer chunks where the LDS still holds
    // the kernel's workgroups: each chunk costs a table build, two barriers
    // and a pass of the fold (the batch-256 decode step's FFN-down, 512x2048
    // CQ2 at 256 activations, 21.5 -> 20.1 us with 8 groups a chunk).
    while (a.gc * 2 <= groups_max &&
           lut_lds_bytes(s0.width, s0.group_bytes, a.gc * 2, kLutTile, a.bpw) <= kLutChunkLds)
        a.gc *= 2;
    // A launch that fills at most a quarter of the CUs is latency-bound: wide
    // rows then take their tables in fewer chunks (up to 64 KiB of tables,
    // all 16 groups of a 4-bit row of 2048 in one chunk of 16 wavefronts),
    // each chunk costing a table build and a barrier.
    if (units * rows * 4 <= device_info().cus)
        while (a.gc * 2 <= groups_max && 2 * a.gc * 2 * s0.group_bytes * 16 * static_cast<int>(sizeof(short)) <= 64 * 1024)
            a.gc *= 2;
    a.bpw_max = a.bpw;
    // Latency-bound launches of one-block units (batch-1 decode) take the
    // wide form: a wavefront per group of the chunk (up to 16), or two per
    // group when the chunk has fewer than 8, so the lookups of one unit
    // spread over more SIMDs.
    a.waves = kLutWaves;
    a.vsplit = 1;
    int gx = wg;
    if (units * rows * 4 <= device_info().cus && a.bpw == 1 && (s0.group_bytes == 32 || s0.group_bytes == 64)) {
        if (a.gc >= 8) {
            a.waves = std::min(16, a.gc);
        } else if (a.gc >= 2) {
            a.waves = 2 * a.gc;
            a.vsplit = 2;
        }
    } else if (s0.group_bytes == 32 || s0.group_bytes == 64) {
        // Launches of up to one workgroup per CU at the widest form also take
        // it: units of bp blocks (the fewest that keep the grid to one
        // round), all the groups in one chunk, a wavefront per (block, group
        // share), up to 16. Each activation's tables are then built once per
        // unit of up to 8 blocks instead of once per unit of the 4-wavefront
        // kernel's 1-2 (measured on MI355X at 256 activations: 512x2048 CQ2
        // with the residual 20.5 -> 17.2 us, 512x512 CQ4 gated with the
        // residual 11.5 -> 10.4 us, 24x2048 CQ4 15.0 -> 9.0 us; at 32-64
        // activations 512x2048 CQ4 15.0 -> 9.1 us, 2048x512 CQ4 8.2 -> 7.5
        // us; bit for bit the same). A grid of more than one round of such
        // workgroups lost (2048x512 CQ4 at 96 activations 16.1 -> 18.2 us).
        int bp = 1;
        const auto grid = [&](int b) {
            long long u = 0;
            for (int k = 0; k < a.njobs; ++k) u += (a.jobs[k].nblk + b - 1) / b;
            return u * rows;
        };
        while (bp < 8 && grid(bp) > device_info().cus) bp *= 2;
        bp = balanced_blocks(nmax, bp);
        int g = groups_max;
        while (g > 1 && lut_lds_bytes(s0.width, s0.group_bytes, g, std::max(kLutTile, bp), bp) > 128 * 1024)
            g = (g + 1) / 2;
        const int waves = std::min(16, bp * g);
        if (grid(bp) <= device_info().cus && waves > kLutWaves) {
            a.waves = waves;
            a.bpw = a.bpw_max = bp;
            a.gc = g;
            a.tb = std::max(kLutTile, bp);
            gx = (nmax + bp - 1) / bp;
        }
    }
    size_t lds = lut_lds_bytes(s0.width, s0.group_bytes, a.gc, a.tb, a.bpw);
    // The next product's tables ride on a launch of one workgroup per
    // activation over all of one view's rows (the wide form), whose
    // workgroups each hold a whole output row.
    if (to && built && a.njobs == 1 && gx == 1 && rows <= 256 && a.waves > kLutWaves && a.vsplit == 1 &&
        s0.group_bytes == s0.width * 16 && a.jobs[0].out == to->in) {
        a.tout = *to;
        lds += lut_tout_lds_bytes(to->in);
        *built = 1;
    }
    for (int r0 = 0; r0 < rows; r0 += 65535) {
        LutLaunch b = a;
        const int nr = std::min(65535, rows - r0);
        for (int k = 0; k < b.njobs; ++k) {
            b.jobs[k].x += static_cast<long long>(r0) * b.jobs[k].x_stride;
            b.jobs[k].y += static_cast<long long>(r0) * b.jobs[k].y_stride;
            if (b.jobs[k].resid) b.jobs[k].resid += static_cast<long long>(r0) * b.jobs[k].resid_stride;
            if (b.jobs[k].xgate) b.jobs[k].xgate += static_cast<long long>(r0) * b.jobs[k].x_stride;
            if (b.jobs[k].app_q) {
                b.jobs[k].app_q += static_cast<long long>(r0) * b.jobs[k].app_q_stride;
                b.jobs[k].app_s += static_cast<long long>(r0) * b.jobs[k].app_s_stride;
                b.jobs[k].app_pos += r0;
            }
        }
        // with the next tables: 256 workgroups, activations spread for the XCDs (the kernel's TB form)
        HIP_TRY(launch_lut(b, s0.width, s0.group_bytes, a.waves, gx, b.tout.tab ? 256 : nr, lds, stream), "lut launch");
    }
    for (int k = 0; k < n; ++k) ms[k]->st->prepared.store(true);
    return CQ_OK;
}

constexpr int kMfmaMinRows = 64;  // activations from which the MFMA form can run
constexpr int kMfmaTile = 64;     // activations per workgroup of the MFMA form (32 when 64 leaves CUs idle)

// The MFMA form pays when its grid fills a good part of the chip; below that
// the lut kernel's workgroup per activation spreads wider.
bool mfma_pays(cq_matrix *const *ms, int n, int rows) {
    if (rows < kMfmaMinRows) return false;
    const int rpw = mfma_rows_per_workgroup() / kBlockRows;
    long long wgs = 0;
    for (int k = 0; k < n; ++k) {
        const int nblk = (ms[k]->row0 + ms[k]->out + kBlockRows - 1) / kBlockRows - ms[k]->row0 / kBlockRows;
        wgs += (nblk + rpw - 1) / rpw;
    }
    wgs *= (rows + kMfmaTile - 1) / kMfmaTile;
    return wgs * 8 >= 3LL * device_info().cus;
}

// One launch of the MFMA form of the lut kernel for up to kKernargJobs views
// of one geometry and the same activations.
int run_mfma(cq_matrix *const *ms, int n, float *const *dsts, const float *x, int rows, hipStream_t stream,
             const Fuse *fz = nullptr) {
    const CqStore &s0 = *ms[0]->st;
    LutLaunch a;
    std::memset(&a, 0, sizeof a);
    const int rpw = mfma_rows_per_workgroup() / kBlockRows;  // blocks per workgroup
    int wg = 0;
    for (int k = 0; k < n; ++k) {
        if (ms[k]->out == 0) continue;
        JobDesc &j = a.jobs[a.njobs];
        fill_job(j, ms[k], x, dsts[k], rows);
        apply_fuse(j, fz, k);
        a.wg0[a.njobs] = wg;
        wg += (j.nblk + rpw - 1) / rpw;
        ++a.njobs;
    }
    if (a.njobs == 0 || rows == 0) return CQ_OK;
    // 32-activation tiles when twice the workgroups of 64 still run in one
    // round on the CUs (2048 rows at 1500 activations: 96 -> 192 workgroups;
    // the 16384-row head at 256: 128 -> 256). A 32-activation workgroup
    // takes about two thirds of a 64-activation one's time (half the MFMAs
    // and table items, one-hot operands reused by one activation tile
    // instead of two), so a second round would lose (512 x 2048 at 12000
    // activations: 482 -> 597 us measured).
    const long long wg64 = static_cast<long long>(wg) * ((rows + kMfmaTile - 1) / kMfmaTile);
    const int ta = 2 * wg64 <= device_info().cus ? kMfmaTile / 2 : kMfmaTile;
    const int max_rows = 65535 * ta;
    for (int r0 = 0; r0 < rows; r0 += max_rows) {
        LutLaunch b = a;
        const int nr = std::min(max_rows, rows - r0);
        for (int k = 0; k < b.njobs; ++k) {
            b.jobs[k].x += static_cast<long long>(r0) * b.jobs[k].x_stride;
            b.jobs[k].y += static_cast<long long>(r0) * b.jobs[k].y_stride;
            if (b.jobs[k].resid) b.jobs[k].resid += static_cast<long long>(r0) * b.jobs[k].resid_stride;
            if (b.jobs[k].xgate) b.jobs[k].xgate += static_cast<long long>(r0) * b.jobs[k].x_stride;
            b.jobs[k].rows = nr;
        }
        HIP_TRY(launch_lut_mfma(b, s0.width, ta, wg, (nr + ta - 1) / ta, stream), "lut mfma launch");
    }
    for (int k = 0; k < n; ++k) ms[k]->st->prepared.store(true);
    return CQ_OK;
}

// ---- workspaces of the table and split forms ----
//
// Both forms keep tables or float terms in device memory between their two
// launches. A product leases a workspace for its launches and returns it
// with an event recorded behind them, in one pool per process that every
// thread shares under a mutex:
// - an idle workspace last used on the same stream is reused at once
//   (stream order protects it); one last used on another stream only once
//   its event has completed; otherwise the product gets a new one, of the
//   size it asks for rounded up to 1 MiB. So products queued at the same
//   time on two streams never share one, from one thread or many;
// - before a new one is allocated, idle workspaces of that device whose
//   work has completed are freed: a device keeps about one workspace per
//   stream with products in flight, each the size of its largest product;
// - a product queued while its stream is captured into a graph leases a
//   workspace of its own, shared only by the products of that capture
//   sequence on that stream (in the graph's order), and never reused or
//   freed: the graph replays it at that address, and the library cannot
//   see when the graph is destroyed. Its allocation is made in relaxed
//   capture mode, so the first product of a shape may be captured.
struct Workspace {
    void *buf = nullptr;
    size_t size = 0;
    int dev = -1;
    hipStream_t stream = nullptr;
    hipEvent_t done = nullptr;  // recorded behind the last lease's launches
    unsigned long long capture = 0;  // capture sequence id of a graph's workspace, 0 otherwise
};

struct WorkspacePool {
    std::mutex mu;
    std::vector<Workspace *> idle;   // eager workspaces not leased
    std::vector<Workspace *> graph;  // held for captured graphs
    size_t held = 0;                 // bytes of all workspaces
};

WorkspacePool &ws_pool() {
    static WorkspacePool *pool = new WorkspacePool;  // never destroyed: graphs may outlive static teardown
    return *pool;
}

constexpr size_t kWsRound = size_t(1) << 20;

struct WsLease {
    Workspace *w = nullptr;
    hipStream_t stream = nullptr;
    bool graph = false;
};

int ws_alloc(Workspace *w, size_t bytes, bool capturing) {
    const size_t want = (std::max<size_t>(bytes, 1) + kWsRound - 1) / kWsRound * kWsRound;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (capturing) HIP_TRY(hipThreadExchangeStreamCaptureMode(&mode), "capture mode");
    const hipError_t e = hipMalloc(&w->buf, want);
    if (capturing) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc workspace");
    w->size = want;
    return CQ_OK;
}

int ws_acquire(size_t bytes, hipStream_t stream, WsLease &l) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev), "current device");
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (stream) HIP_TRY(hipStreamGetCaptureInfo(stream, &cs, &cid), "capture info");
    WorkspacePool &p = ws_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    l.stream = stream;
    if (cs == hipStreamCaptureStatusActive) {
        l.graph = true;
        Workspace *best = nullptr;
        for (Workspace *w : p.graph)
            if (w->dev == dev && w->capture == cid && w->stream == stream && w->size >= bytes &&
                (!best || w->size < best->size))
                best = w;
        if (!best) {
            std::unique_ptr<Workspace> w(new Workspace);
            if (int e = ws_alloc(w.get(), bytes, true)) return e;
            w->dev = dev;
            w->stream = stream;
            w->capture = cid;
            p.held += w->size;
            best = w.release();
            p.graph.push_back(best);
        }
        l.w = best;
        return CQ_OK;
    }
    // An idle workspace of this device: one last used on this stream first,
    // else one whose work has completed.
    int pick = -1;
    for (size_t i = 0; i < p.idle.size(); ++i) {
        Workspace *w = p.idle[i];
        if (w->dev != dev || w->size < bytes) continue;
        if (w->stream == stream) {
            pick = static_cast<int>(i);
            break;
        }
        if (pick < 0 && hipEventQuery(w->done) == hipSuccess) pick = static_cast<int>(i);
    }
    if (pick >= 0) {
        l.w = p.idle[pick];
        p.idle.erase(p.idle.begin() + pick);
        return CQ_OK;
    }
    // None fits: free this device's completed idle workspaces (all smaller
    // than the request, or busy on other streams), then allocate.
    for (size_t i = 0; i < p.idle.size();) {
        Workspace *w = p.idle[i];
        if (w->dev == dev && hipEventQuery(w->done) == hipSuccess) {
            (void)hipEventDestroy(w->done);
            (void)hipFree(w->buf);
            p.held -= w->size;
            delete w;
            p.idle.erase(p.idle.begin() + i);
        } else {
            ++i;
        }
    }
    std::unique_ptr<Workspace> w(new Workspace);
    if (int e = ws_alloc(w.get(), bytes, false)) return e;
    // Device scope is enough for this event: it only tells when the lease's
    // kernels are done with the buffer, for reuse on another stream of the
    // same device or hipFree; a system-scope fence behind every eager
    // product would write back the L2s between two launches.
    const hipError_t e = hipEventCreateWithFlags(&w->done, hipEventDisableTiming | hipEventDisableSystemFence);
    if (e != hipSuccess) {
        (void)hipFree(w->buf);
        return hip_fail(e, "workspace event");
    }
    w->dev = dev;
    p.held += w->size;
    l.w = w.release();
    return CQ_OK;
}

// Returns a lease after its launches were queued (or failed to queue).
int ws_release(WsLease &l) {
    if (!l.w || l.graph) return CQ_OK;
    Workspace *w = l.w;
    l.w = nullptr;
    const hipError_t e = hipEventRecord(w->done, l.stream);
    WorkspacePool &p = ws_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    if (e != hipSuccess) {  // nothing marks its last use: keep it out of reuse
        p.graph.push_back(w);
        return hip_fail(e, "workspace event record");
    }
    w->stream = l.stream;
    p.idle.push_back(w);
    return CQ_OK;
}

// Holds a lease for the scope of one product.
struct WsScope {
    WsLease l;
    ~WsScope() { (void)ws_release(l); }
};

constexpr int kSplitMinRows = 320;  // activations from which the split form pays

// The split form pays where the 512-row MFMA form leaves CUs idle and the
// lut kernel repeats every table lookup per activation: some hundreds of
// activations or more (measured on MI355X: 375 and 1500 encoder frames of
// 512x2048 CQ4 52 -> 40 us and 142 -> 86 us, 2048x512 CQ4 at 375 46 -> 40
// us). At the decode step's 256 activations its workgroups (one wavefront
// per SIMD, tables and one-hot operands built per 32 activations) lose to
// the lut kernel (a 512x512 CQ4 product 12 -> 28 us), and so do 2-bit
// products of four groups (2048x512 CQ2 at 375: 27 -> 30 us). Its grid
// (256-row tiles x 32-activation tiles x groups) must also reach a quarter
// of the CUs.
bool split_pays(cq_matrix *const *ms, int n, int rows) {
    if (rows < kSplitMinRows || n > kKernargJobs) return false;
    const CqStore &s0 = *ms[0]->st;
    if (!mfma_geometry_supported(s0.width, s0.group)) return false;
    if (s0.width == 2 && s0.groups <= 4) return false;
    const int rpw = mfma_split_rows_per_workgroup() / kBlockRows;
    long long wgs = 0;
    for (int k = 0; k < n; ++k) {
        if (!uses_lut(ms[k])) return false;
        const int nblk = (ms[k]->row0 + ms[k]->out + kBlockRows - 1) / kBlockRows - ms[k]->row0 / kBlockRows;
        wgs += (nblk + rpw - 1) / rpw;
    }
    const int ta = mfma_split_activations();
    wgs *= static_cast<long long>((rows + ta - 1) / ta) * s0.groups;
    return 4 * wgs >= device_info().cus;
}

int run_split(cq_matrix *const *ms, int n, float *const *dsts, const float *x, int rows, hipStream_t stream,
              const Fuse *fz = nullptr) {
    const CqStore &s0 = *ms[0]->st;
    const int ta = mfma_split_activations();
    const int rpw = mfma_split_rows_per_workgroup() / kBlockRows;
    const int max_rows = 65535 * 4;  // the fold's grid y: activations in fours
    for (int r0 = 0; r0 < rows; r0 += max_rows) {
        const int nr = std::min(max_rows, rows - r0);
        LutLaunch a;
        std::memset(&a, 0, sizeof a);
        int wg = 0, fold = 0;
        size_t terms = 0;
        for (int k = 0; k < n; ++k) {
            if (ms[k]->out == 0) continue;
            JobDesc &j = a.jobs[a.njobs];
            fill_job(j, ms[k], x + static_cast<long long>(r0) * s0.in, dsts[k] + static_cast<long long>(r0) * ms[k]->out,
                     nr);
            apply_fuse(j, fz, k);
            if (j.resid) j.resid += static_cast<long long>(r0) * j.resid_stride;
            if (j.xgate) j.xgate += static_cast<long long>(r0) * j.x_stride;
            if (j.app_q) {
                j.app_q += static_cast<long long>(r0) * j.app_q_stride;
                j.app_s += static_cast<long long>(r0) * j.app_s_stride;
                j.app_pos += r0;
            }
            a.wg0[a.njobs] = wg;
            a.fold0[a.njobs] = fold;
            wg += (j.nblk + rpw - 1) / rpw;
            fold += (j.nblk + 3) / 4;  // the fold's workgroups cover 256 rows
            terms += static_cast<size_t>(j.groups) * nr * j.nblk * kBlockRows;
            ++a.njobs;
        }
        if (a.njobs == 0 || nr == 0) return CQ_OK;
        a.split_at = (nr + ta - 1) / ta;
        a.split_tiles = wg * a.split_at;
        WsScope ws;
        if (int e = ws_acquire(terms * sizeof(float), stream, ws.l)) return e;
        float *const base = static_cast<float *>(ws.l.w->buf);
        size_t off = 0;
        for (int k = 0; k < a.njobs; ++k) {
            a.term[k] = base + off;
            off += static_cast<size_t>(a.jobs[k].groups) * nr * a.jobs[k].nblk * kBlockRows;
        }
        HIP_TRY(launch_lut_mfma_split(a, s0.width, fold, stream), "lut mfma split launch");
        if (int e = ws_release(ws.l)) return e;
    }
    for (int k = 0; k < n; ++k) ms[k]->st->prepared.store(true);
    return CQ_OK;
}

// ---- the table form ----
//
// A pre-pass builds each activation's tables once and the MFMAs of every
// 64-row block stream them. A workgroup reads its 32 activations' tables
// whole (16 KiB per activation and 512 inputs), so the form pays where the
// lut kernel's work, linear in rows x activations, outgrows the form's
// ~15 us floor at these sizes (from about 256K row-activations at 4 bits,
// 384K at 2, and 16 activations), or where its (block, tile) workgroups
// reach the CUs; past 3072 activations over 768 rows or more, at 2 bits,
// or up to 6144 activations (a 512-row CQ4 matrix's tables, read by few
// blocks, cost more than the 512-row MFMA form's own table builds at 12000).
// Measured on MI355X (pre-pass + product against the form chosen
// otherwise): at 256 activations the four 512x512 CQ4 q/k/v/gate products
// with the norm 18.6 against 28.2 us, 2048x512 CQ2 with the norm and SiLU
// 16.0 against 19.1 us, the 16384x512 head 60.2 against 64.4 us, 1536x512
// CQ4 16.2 against 23.5 us, 1024x512 CQ4 15.9 against 16.7 us, but 1024x512
// CQ2 12.0 against 10.8 us and a 512x512 CQ4 product 14.9 against 9.6 us;
// the 16384x512 CQ4 head at 16, 32, 64 and 95 activations 15.5, 15.7, 22.6,
// 30.3 us against 16.8, 28.0, 50.4, 70.1 us (CQ2 at 32 and 64 12.1 and 16.0
// against 17.7 and 30.4 us);
// 2048x512 CQ4 at 64, 96, 192 activations 14.7, 16.1, 17.5 us against the
// lut kernel's 10.8, 17.0, 26.8 us; at 375, 1024, 1500, 3000, 6000 and
// 12000 activations 25.8, 44.0, 57.5, 107.1, 194.4, 361.1 us against 31.4,
// 57.7, 67.5, 118.0, 244.0, 363.8 us (split, split, then the 512-row MFMA
// form), CQ2 at 375, 1500, 6000, 12000 16.9, 36.7, 106.7, 203.4 against
// 25.5, 43.9, 154.3, 236.1 us; 1024x512 CQ4 at 1500, 6000, 12000 37.5,
// 101.7, 202.2 us against 43.2, 114.4, 220.3 us; 512x512 CQ4 at 12000 120.3
// against the MFMA form's 111.4 us, but at 4000 and 6000 activations 50.9
// and 68.5 us against the split form's 53.8 and 75.3 us (CQ2 at 4000, 6000,
// 12000: 35.8, 45.6, 73.9 against 52.8, 74.8, 83.8 us); 768x512 CQ4 at 4000,
// 6000, 12000 62.2, 85.7, 162.6 us against the MFMA form's 70.2, 117.9,
// 225.6 us; small matrices past 3072 activations keep the form at 2 bits
// (64x512 CQ2 at 3500 / 12000: 23.5 / 40.8 against the MFMA form's 40.5 /
// 77.3 us, 384x512 CQ2 at 12000 70.1 against 79.0 us) and at 4 bits to
// 6144 (64x512 CQ4 at 6000: 40.2 against 62.4 us; at 12000 the two are
// within 1%). The views must share their tables (one
// pre-pass serves them all). The tables live in a leased workspace (at 12288
// activations of 1024 inputs, 384 MiB).
constexpr int kTabMinRows = 16;
constexpr int kTabMaxRows = 3072;       // any row count
constexpr int kTabMaxRowsWide = 12288;  // over kTabWideBlocks blocks, at 2 bits, or to kTabMidRows
constexpr int kTabWideBlocks = 12;
constexpr int kTabMidRows = 6144;
constexpr long long kTabMinWork4 = 256LL * 1024;  // rows x activations, 4-bit
constexpr long long kTabMinWork2 = 384LL * 1024;  // rows x activations, 2-bit
constexpr int kTabMaxGroups = 8;

bool tab_pays(cq_matrix *const *ms, int n, int rows) {
    if (rows < kTabMinRows || rows > kTabMaxRowsWide || n > kKernargJobs) return false;
    const CqStore &s0 = *ms[0]->st;
    if (!mfma_geometry_supported(s0.width, s0.group) || s0.groups > std::min(kTabMaxGroups, tab_max_groups()))
        return false;
    long long blocks = 0;
    for (int k = 0; k < n; ++k) {
        if (!uses_lut(ms[k]) || !shares_tables(s0, *ms[k]->st)) return false;
        blocks += (ms[k]->row0 + ms[k]->out + kBlockRows - 1) / kBlockRows - ms[k]->row0 / kBlockRows;
    }
    if (rows > kTabMaxRows) return blocks >= kTabWideBlocks || s0.width == 2 || rows <= kTabMidRows;
    const long long work = blocks * 64LL * rows;  // in whole 64-row blocks
    return work >= (s0.width == 4 ? kTabMinWork4 : kTabMinWork2) || blocks * ((rows + 31) / 32) >= device_info().cus;
}

// Row blocks per workgroup of the table form's product: slabs of 4 blocks
// whose wavefronts share the tile's A operands through LDS (a quarter of the
// L2 reads) once such workgroups number two per CU or more; below that the
// workgroup per block spreads wider. Measured on MI355X (one block, against
// four): 2048x512 CQ4 at 6000 and 12000 activations 188.4 / 359.7 -> 179.5 /
// 332.2 us, 2048x1024 CQ4 at 12000 809 -> 615 us, the 16384x512 head at 256,
// 1500 and 12000 66.8 / 315.7 / 2433 -> 64.5 / 297.3 / 2137 us; 2048x512
// CQ4 at 1500 (376 slab workgroups) 60.0 -> 66.9 us and at 256 (64) 16.4
// -> 38.3 us.
int tab_row_blocks(cq_matrix *const *ms, int n, int rows) {
    long long slabs = 0;
    for (int k = 0; k < n; ++k) {
        const int nblk = (ms[k]->row0 + ms[k]->out + kBlockRows - 1) / kBlockRows - ms[k]->row0 / kBlockRows;
        if (ms[k]->out > 0) slabs += (nblk + 3) / 4;
    }
    return slabs * ((rows + 31) / 32) >= 2LL * device_info().cus ? 4 : 1;
}

int run_tab(cq_matrix *const *ms, int n, float *const *dsts, const float *x, int rows, hipStream_t stream,
            const Fuse *fz = nullptr, const void *tables = nullptr) {
    const CqStore &s0 = *ms[0]->st;
    LutLaunch a;
    std::memset(&a, 0, sizeof a);
    const int rb = tab_row_blocks(ms, n, rows);
    int blocks = 0;  // slabs of rb row blocks
    for (int k = 0; k < n; ++k) {
        if (ms[k]->out == 0) continue;
        JobDesc &j = a.jobs[a.njobs];
        fill_job(j, ms[k], x, dsts[k], rows);
        apply_fuse(j, fz, k);
        a.wg0[a.njobs] = blocks;
        blocks += (j.nblk + rb - 1) / rb;
        ++a.njobs;
    }
    if (a.njobs == 0 || rows == 0) return CQ_OK;
    a.tab_rb = rb;
    const int tiles = (rows + 31) / 32;
    TabArgs t;
    std::memset(&t, 0, sizeof t);
    t.x = x;
    t.x_stride = s0.in;
    t.xgate = a.jobs[0].xgate;
    t.ngain = a.jobs[0].ngain;
    t.rows = rows;
    t.in = s0.in;
    t.groups = s0.groups;
    t.tiles = tiles;
    for (int c = 0; c < 16; ++c) t.cb[c] = a.jobs[0].cb[c];
    t.cb_max = s0.cb_max;
    t.lut_step = s0.lut_step;
    const size_t tb = tab_table_bytes(s0.width, s0.groups, tiles), sb = tab_step_bytes(s0.groups, tiles);
    WsScope ws;
    char *base = static_cast<char *>(const_cast<void *>(tables));
    if (!base) {
        if (int e = ws_acquire(tb + sb, stream, ws.l)) return e;
        base = static_cast<char *>(ws.l.w->buf);
    }
    t.tab = reinterpret_cast<int8_t *>(base);
    t.stp = reinterpret_cast<float *>(base + tb);
    a.tab = t.tab;
    a.tstp = t.stp;
    a.tab_at = tiles;
    a.tab_nb = blocks;
    HIP_TRY(launch_lut_tab(t, a, s0.width, blocks, stream, tables == nullptr), "lut table-form launch");
    if (int e = ws_release(ws.l)) return e;
    for (int k = 0; k < n; ++k) ms[k]->st->prepared.store(true);
    return CQ_OK;
}

// Launches the product of up to kMaxMatrices views sharing their tables.
// ---- the dense form of Dense views ----

// Activations from which a Dense view's product runs the fp32 MFMA form;
// fewer run Exact's nibble kernels, whose result (bit for bit Exact's) is
// within the same bound.
constexpr int kDenseMinRows = 16;

bool dense_pays(cq_matrix *const *ms, int n, int rows) {
    if (rows < kDenseMinRows) return false;
    const CqStore &s0 = *ms[0]->st;
    if (!dense_geometry_supported(s0.width, s0.group)) return false;
    for (int k = 0; k < n; ++k)
        if (!ms[k]->dense || ms[k]->st->group != s0.group || ms[k]->st->groups != s0.groups ||
            ms[k]->st->width != s0.width)
            return false;
    return true;
}

// K runs of a view's dense product, chosen by a cost model: its items
// (128 x 128 tiles x runs) go round the CUs, two resident on a CU at a
// time, and a CU works through its ceil(items / CUs) items at about 4 us a
// chunk of 64 coordinates (measured on MI355X: a CU holding two items takes
// about twice as long as one holding one); more than one run adds the
// partial sums' traffic (each run writes rows x out floats, the fold reads
// them all and writes y once, at about 4 TB/s) and a launch.
void dense_split(int tiles, int nch, int rows, int out, int &ksplit, int &kchunks) {
    const long long slots = device_info().cus;
    double best = 0;
    ksplit = 1;
    for (int ks = 1; ks <= nch; ++ks) {
        const int kc = (nch + ks - 1) / ks;
        if ((nch + kc - 1) / kc != ks) continue;  // the same runs as a smaller count
        const long long items = static_cast<long long>(tiles) * ks;
        double us = static_cast<double>((items + slots - 1) / slots) * kc * 4.0;
        if (ks > 1) us += (2.0 * ks + 1) * rows * static_cast<double>(out) * 4 / 4e6 + 3.0;
        if (ks == 1 || us < best) best = us, ksplit = ks;
    }
    kchunks = (nch + ksplit - 1) / ksplit;
}

// One rotation of the activations into a workspace, then one product launch
// (and its fold) per view.
int run_dense(cq_matrix *const *ms, int n, float *const *dsts, const float *x, int rows, hipStream_t stream) {
    const CqStore &s0 = *ms[0]->st;
    const int tn = dense_tile_activations(), tmr = dense_tile_rows() / kBlockRows;
    const int kin = s0.groups * s0.group, kpad = (kin + 63) / 64 * 64, nch = kpad / 64;
    const int tiles_n = (rows + tn - 1) / tn;
    size_t part = 0;
    for (int k = 0; k < n; ++k) {
        const int nblk = (ms[k]->row0 + ms[k]->out + kBlockRows - 1) / kBlockRows - ms[k]->row0 / kBlockRows;
        int ks, kc;
        dense_split(((nblk + tmr - 1) / tmr) * tiles_n, nch, rows, ms[k]->out, ks, kc);
        if (ks > 1) part = std::max(part, static_cast<size_t>(ks) * rows * ms[k]->out * sizeof(float));
    }
    DenseRotArgs r;
    std::memset(&r, 0, sizeof r);
    r.x = x;
    r.x_stride = s0.in;
    r.rows = rows;
    r.rows_pad = tiles_n * tn;
    r.in = s0.in;
    r.G = s0.group;
    r.groups = s0.groups;
    r.kpad = kpad;
    r.inv_sqrt = s0.inv_sqrt;
    const size_t xh_bytes = align256(static_cast<size_t>(r.rows_pad) * kpad * sizeof(float));
    WsScope ws;
    if (int e = ws_acquire(xh_bytes + part, stream, ws.l)) return e;
    r.xh = static_cast<float *>(ws.l.w->buf);
    HIP_TRY(launch_dense_rotate(r, stream), "dense rotation launch");
    for (int k = 0; k < n; ++k) {
        const cq_matrix *m = ms[k];
        if (m->out == 0) continue;
        const CqStore &s = *m->st;
        DenseArgs a;
        std::memset(&a, 0, sizeof a);
        a.idx = s.d_idx;
        a.norm = s.d_norm;
        a.xh = r.xh;
        a.y = dsts[k];
        a.part = reinterpret_cast<float *>(static_cast<char *>(ws.l.w->buf) + xh_bytes);
        a.y_stride = m->out;
        a.row0 = m->row0;
        a.out = m->out;
        a.blk0 = m->row0 / kBlockRows;
        a.nblk = (m->row0 + m->out + kBlockRows - 1) / kBlockRows - a.blk0;
        a.rows = rows;
        a.kpad = kpad;
        a.kin = kin;
        a.groups = s.groups;
        a.G = s.group;
        a.U = s.unit_bytes;
        a.units = s.units;
        a.tiles_m = (a.nblk + tmr - 1) / tmr;
        a.tiles_n = tiles_n;
        dense_split(a.tiles_m * a.tiles_n, nch, rows, a.out, a.ksplit, a.kchunks);
        for (int c = 0; c < 16; ++c) a.cb[c] = c < s.ncb ? s.cb[c] : 0.0f;
        HIP_TRY(launch_dense(a, s.width, stream), "dense product launch");
    }
    return ws_release(ws.l);
}

int run_product(cq_matrix *const *ms, int n, float *const *dsts, const float *x, int rows, hipStream_t stream,
                const Fuse *fz = nullptr, const TabOut *to = nullptr, int *built = nullptr) {
    const CqStore &s0 = *ms[0]->st;
    const int mode = uses_lut(ms[0]) ? kModeLut : kModeExact;
    if (mode == kModeLut && tab_pays(ms, n, rows)) return run_tab(ms, n, dsts, x, rows, stream, fz);
    if (mode == kModeLut && n <= kKernargJobs && mfma_geometry_supported(s0.width, s0.group) &&
        mfma_pays(ms, n, rows))
        return run_mfma(ms, n, dsts, x, rows, stream, fz);
    if (mode == kModeLut && split_pays(ms, n, rows)) return run_split(ms, n, dsts, x, rows, stream, fz);
    if (mode == kModeLut && lut_fits(s0) && n <= kKernargJobs)
        return run_lut(ms, n, dsts, x, rows, stream, fz, to, built);
    if (fz && fz->any())
        return fail(CQ_ERR_UNSUPPORTED, "cq: fused products run the lut kernel (this is %s, group bytes %d)",
                    mode == kModeLut ? "lut" : "exact", s0.group_bytes);
    if (ms[0]->dense && dense_pays(ms, n, rows)) return run_dense(ms, n, dsts, x, rows, stream);
    int rc = check_geometry(s0, mode);
    if (rc) return rc;
    ProdArgs a;
    std::memset(&a, 0, sizeof a);
    fill_common(a, s0, rows);
    a.x = x;
    a.x_stride = s0.in;
    long long nblk_total = 0;
    for (int k = 0; k < n; ++k) {
        const int row0 = ms[k]->row0, out = ms[k]->out;
        nblk_total += (row0 + out + kBlockRows - 1) / kBlockRows - row0 / kBlockRows;
    }
    LaunchPlan p = plan(s0, mode, nblk_total, rows);
    if (p.lds > device_info().max_lds)
        return fail(CQ_ERR_UNSUPPORTED, "cq: a product of group %d needs %zu bytes of LDS", s0.group, p.lds);
    a.tb = p.tb;
    a.gc = p.gc;
    int tiles = 0;
    a.nmats = 0;
    for (int k = 0; k < n; ++k) {
        const cq_matrix *m = ms[k];
        if (m->out == 0) continue;
        MatDesc &d = a.mats[a.nmats++];
        d.idx = m->st->d_idx;
        d.norm = m->st->d_norm;
        d.y = dsts[k];
        d.y_stride = m->out;
        d.row0 = m->row0;
        d.out = m->out;
        d.blk0 = m->row0 / kBlockRows;
        d.tile0 = tiles;
        const int nb = (m->row0 + m->out + kBlockRows - 1) / kBlockRows - d.blk0;
        tiles += (nb + p.tb - 1) / p.tb;
    }
    a.tiles = tiles;
    if (a.nmats == 0 || rows == 0) return CQ_OK;
    HIP_TRY(launch_product(a, s0.width, s0.group_bytes, mode, p.lds, stream), "product launch");
    if (mode == kModeLut)
        for (int k = 0; k < n; ++k) ms[k]->st->prepared.store(true);
    return CQ_OK;
}

// cq.GEMMs on device pointers: one launch per run of up to kMaxMatrices
// matrices that share their tables and kernel, else one launch per matrix
// (each gives the same bits either way: kernel.go:127-133).
int gemms_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows, hipStream_t stream,
              const Fuse *fz = nullptr) {
    int k = 0;
    while (k < n) {
        int e = k + 1;
        while (e < n && e - k < kMaxMatrices && uses_lut(ms[e]) == uses_lut(ms[k]) && ms[e]->dense == ms[k]->dense &&
               shares_tables(*ms[k]->st, *ms[e]->st))
            ++e;
        int rc = run_product(ms + k, e - k, dsts + k, x, rows, stream, fz);
        if (rc) return rc;
        k = e;
    }
    return CQ_OK;
}

int row_args(const cq_matrix *m, RowArgs &a) {
    const CqStore &s = *m->st;
    std::memset(&a, 0, sizeof a);
    a.idx = s.d_idx;
    a.norm = s.d_norm;
    a.in = s.in;
    a.group = s.group;
    a.groups = s.groups;
    a.row_bytes = s.row_bytes;
    a.width = s.width;
    a.units = s.units;
    a.unit_bytes = s.unit_bytes;
    for (int c = 0; c < 16; ++c) a.cb[c] = c < s.ncb ? s.cb[c] : 0.0f;
    a.inv_sqrt = s.inv_sqrt;
    a.nrows = s.out;
    a.scale = 1.0f;
    if (static_cast<size_t>(s.group) * 4 > device_info().max_lds)
        return fail(CQ_ERR_UNSUPPORTED, "cq: Row of group %d", s.group);
    return CQ_OK;
}

}  // namespace

// ---- C ABI -----------------------------------------------------------------

extern "C" {

const char *cq_last_error(void) { return t_err.c_str(); }

const char *cq_version(void) { return "libcqhip 0.1 (gfx950)"; }

int cq_device_info(char *buf, size_t len) {
    const DeviceInfo &d = device_info();
    if (d.device < 0) return fail(CQ_ERR_DEVICE, "cq: no HIP device");
    if (buf && len)
        snprintf(buf, len, "device %d %s, %d CUs, %zu bytes LDS per workgroup; kernels: lut, nibble4, nibble, row, "
                 "int8 quantize, int8 attend", d.device, d.name.c_str(), d.cus, d.max_lds);
    return CQ_OK;
}

int cq_new(int out, int in, int group, int bits, int width, const float *codebook, size_t codebook_len,
           const uint8_t *index, size_t index_len, const uint8_t *norms_fp16, size_t norms_len, int gather,
           cq_matrix **mp) {
    if (!mp) return fail(CQ_ERR_MISUSE, "cq: nil result pointer");
    *mp = nullptr;
    // internal/cq/matrix.go:61-73, in the reference's order.
    if ((bits != 2 && bits != 4) || width != bits)
        return fail(CQ_ERR_ARG, "cq: %d-bit CQ (index width %d) not supported, only 2 and 4", bits, width);
    if (group < 8 || (group & (group - 1)) != 0)
        return fail(CQ_ERR_ARG, "cq: group %d is not a power of two >= 8", group);
    if (out < 0 || in <= 0) return fail(CQ_ERR_ARG, "cq: bad shape [%d, %d]", out, in);
    if (codebook_len != (static_cast<size_t>(1) << bits))
        return fail(CQ_ERR_ARG, "cq: %zu codebook levels for %d bits", codebook_len, bits);
    const int groups = (in + group - 1) / group;
    const long long row_bytes = static_cast<long long>(groups) * group * width / 8;
    if (index_len != static_cast<size_t>(out) * row_bytes || norms_len != 2 * static_cast<size_t>(out) * groups)
        return fail(CQ_ERR_ARG, "cq: %zu index and %zu norm bytes for [%d, %d], want %lld and %lld", index_len,
                    norms_len, out, in, static_cast<long long>(out) * row_bytes, 2LL * out * groups);
    if (device_info().device < 0) return fail(CQ_ERR_DEVICE, "cq: no HIP device");

    auto st = std::make_shared<CqStore>();
    st->out = out;
    st->in = in;
    st->group = group;
    st->groups = groups;
    st->width = width;
    st->row_bytes = static_cast<int>(row_bytes);
    st->group_bytes = group * width / 8;
    st->unit_bytes = std::min(16, st->group_bytes);
    st->units = st->row_bytes / st->unit_bytes;
    st->nblk = (out + kBlockRows - 1) / kBlockRows;
    st->ncb = 1 << bits;
    st->cb_max = 0;
    for (int c = 0; c < st->ncb; ++c) {
        st->cb[c] = codebook[c];
        st->cb_max = gomax(st->cb_max, std::fabs(codebook[c]));
    }
    st->lut_step = static_cast<float>(1.0 / (kLutQ * std::sqrt(static_cast<double>(group))));  // lut.go:213-215
    st->inv_sqrt = static_cast<float>(1.0 / std::sqrt(static_cast<double>(group)));          // kernel.go:377

    // Device layout (cq_internal.hpp): blocks of 64 rows, units side by side.
    const size_t nrows = static_cast<size_t>(std::max(st->nblk, 1)) * kBlockRows;
    st->idx_bytes = nrows * st->row_bytes;
    st->norm_bytes = nrows * groups * sizeof(uint16_t);
    if (st->idx_bytes > static_cast<size_t>(INT32_MAX))  // the lut kernel's buffer loads take 32-bit offsets
        return fail(CQ_ERR_UNSUPPORTED, "cq: %zu index bytes (this library holds at most 2 GiB per matrix)",
                    st->idx_bytes);
    std::vector<uint8_t> hidx(st->idx_bytes, 0);
    std::vector<uint16_t> hnorm(nrows * groups, 0);
    const int U = st->unit_bytes;
    for (int r = 0; r < out; ++r) {
        const size_t blk = r / kBlockRows, lane = r % kBlockRows;
        const uint8_t *src = index + static_cast<size_t>(r) * row_bytes;
        for (int u = 0; u < st->units; ++u)
            std::memcpy(&hidx[((blk * st->units + u) * kBlockRows + lane) * U], src + static_cast<size_t>(u) * U, U);
        for (int g = 0; g < groups; ++g) {
            const uint8_t *nb = norms_fp16 + 2 * (static_cast<size_t>(r) * groups + g);
            hnorm[(blk * groups + g) * kBlockRows + lane] = static_cast<uint16_t>(nb[0] | (nb[1] << 8));
        }
    }
    HIP_TRY(hipMalloc(&st->d_idx, align256(st->idx_bytes)), "hipMalloc index");
    HIP_TRY(hipMalloc(&st->d_norm, align256(st->norm_bytes)), "hipMalloc norms");
    HIP_TRY(hipMemcpy(st->d_idx, hidx.data(), st->idx_bytes, hipMemcpyHostToDevice), "upload index");
    HIP_TRY(hipMemcpy(st->d_norm, hnorm.data(), st->norm_bytes, hipMemcpyHostToDevice), "upload norms");

    auto *m = new cq_matrix{st, 0, out, false};
    if (!gather && uses_lut(m)) st->prepared.store(true);  // New = NewGather + Prepare (matrix.go:46-55)
    *mp = m;
    return CQ_OK;
}

void cq_free(cq_matrix *m) { delete m; }

int cq_out(const cq_matrix *m) { return m ? m->out : 0; }
int cq_in(const cq_matrix *m) { return m ? m->st->in : 0; }
int cq_bits(const cq_matrix *m) { return m ? m->st->width : 0; }

int cq_prepare(cq_matrix *m) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (uses_lut(m)) m->st->prepared.store(true);  // matrix.go:111-115
    return CQ_OK;
}

long long cq_bytes(const cq_matrix *m) {
    // matrix.go:121-129: packed index + float32 norms + codebook, and the
    // lut copy of the view's 32-row blocks once built (lut.go:82-86).
    if (!m) return 0;
    const CqStore &s = *m->st;
    long long n = static_cast<long long>(m->out) * s.row_bytes + 4LL * m->out * s.groups + 4LL * s.ncb;
    if (uses_lut(m) && s.prepared.load()) {
        const long long b0 = m->row0 / 32, b1 = (m->row0 + m->out + 31) / 32;
        n += (b1 - b0) * 32 * (s.row_bytes + 4LL * s.groups);
    }
    return n;
}

long long cq_device_bytes(const cq_matrix *m) {
    return m ? static_cast<long long>(m->st->idx_bytes + m->st->norm_bytes) : 0;
}

int cq_rows(const cq_matrix *m, int lo, int hi, cq_matrix **view) {
    if (!m || !view) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (lo < 0 || hi < lo || hi > m->out) return fail(CQ_ERR_MISUSE, "cq: Rows(%d, %d) of %d rows", lo, hi, m->out);
    *view = new cq_matrix{m->st, m->row0 + lo, hi - lo, m->exact, m->dense};
    return CQ_OK;
}

int cq_exact(const cq_matrix *m, cq_matrix **view) {
    if (!m || !view) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    *view = new cq_matrix{m->st, m->row0, m->out, true};
    return CQ_OK;
}

int cq_dense(const cq_matrix *m, cq_matrix **view) {
    if (!m || !view) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    *view = new cq_matrix{m->st, m->row0, m->out, true, true};
    return CQ_OK;
}

const char *cq_kernel_name(const cq_matrix *m) {
    if (m && m->dense) return "dense-f32";
    return m && uses_lut(m) ? "lut" : "nibble4";
}

int cq_gemm_mfma_dev(const cq_matrix *m, float *dst, const float *x, int rows, void *stream) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (rows < 0) return fail(CQ_ERR_MISUSE, "cq: GEMM of %d rows", rows);
    if (!uses_lut(m) || !mfma_geometry_supported(m->st->width, m->st->group))
        return fail(CQ_ERR_UNSUPPORTED, "cq: the MFMA form needs a lut matrix of group 128 (group %d, %s)",
                    m->st->group, m->exact ? "exact" : "lut");
    if (rows == 0 || m->out == 0) return CQ_OK;
    if (!dst || !x) return fail(CQ_ERR_MISUSE, "cq: nil device pointer");
    cq_matrix *mm = const_cast<cq_matrix *>(m);
    return run_mfma(&mm, 1, &dst, x, rows, static_cast<hipStream_t>(stream));
}

const char *cq_gemm_path(const cq_matrix *m, int rows) {
    cq_matrix *mm = const_cast<cq_matrix *>(m);
    if (m && m->dense && dense_pays(&mm, 1, rows)) return "dense-f32";
    if (!m || !uses_lut(m)) return "nibble4";
    if (tab_pays(&mm, 1, rows)) return "lut-mfma-tab";
    if (mfma_geometry_supported(m->st->width, m->st->group) && mfma_pays(&mm, 1, rows)) return "lut-mfma";
    if (split_pays(&mm, 1, rows)) return "lut-mfma-split";
    return "lut";
}

int cq_gemm_dev(const cq_matrix *m, float *dst, const float *x, int rows, void *stream) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (rows < 0) return fail(CQ_ERR_MISUSE, "cq: GEMM of %d rows", rows);
    if (rows == 0 || m->out == 0) return CQ_OK;  // kernel.go:105-107
    if (!dst || !x) return fail(CQ_ERR_MISUSE, "cq: GEMM of %d rows with a nil operand", rows);
    cq_matrix *mm = const_cast<cq_matrix *>(m);
    return run_product(&mm, 1, &dst, x, rows, static_cast<hipStream_t>(stream));
}

// Nil operands of a device product: a nil Go slice reaches the C ABI as a
// null pointer, which must not reach a kernel.
static int nil_operands(int n, float *const *dsts, const float *x, int rows) {
    if (rows == 0 || n == 0) return CQ_OK;
    if (!x) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d rows with a nil input", rows);
    for (int k = 0; k < n; ++k)
        if (!dsts[k]) return fail(CQ_ERR_MISUSE, "cq: GEMMs with a nil output %d", k);
    return CQ_OK;
}

long long cq_workspace_held(void) {
    WorkspacePool &p = ws_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    return static_cast<long long>(p.held);
}

long long cq_workspace_trim(void) {
    WorkspacePool &p = ws_pool();
    std::lock_guard<std::mutex> lock(p.mu);
    for (size_t i = 0; i < p.idle.size();) {
        Workspace *w = p.idle[i];
        if (hipEventQuery(w->done) == hipSuccess) {
            (void)hipEventDestroy(w->done);
            (void)hipFree(w->buf);
            p.held -= w->size;
            delete w;
            p.idle.erase(p.idle.begin() + i);
        } else {
            ++i;
        }
    }
    return static_cast<long long>(p.held);
}

int cq_gemms_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows, void *stream) {
    if (n < 0 || (n > 0 && (!ms || !dsts))) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d matrices", n);
    if (rows < 0) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d rows", rows);
    for (int k = 0; k < n; ++k)
        if (!ms[k] || ms[k]->st->in != ms[0]->st->in)
            return fail(CQ_ERR_MISUSE, "cq: GEMMs over matrices of different input widths");
    if (int e = nil_operands(n, dsts, x, rows)) return e;
    if (rows == 0 || n == 0) return CQ_OK;
    return gemms_dev(n, ms, dsts, x, rows, static_cast<hipStream_t>(stream));
}

int cq_gemms_fused_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows,
                       const float *norm_gain, const float *resid, int act, void *stream) {
    if (n < 0 || (n > 0 && (!ms || !dsts))) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d matrices", n);
    if (rows < 0) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d rows", rows);
    if (act != 0 && act != 1) return fail(CQ_ERR_MISUSE, "cq: activation %d", act);
    if (resid && (n != 1 || act != 0))
        return fail(CQ_ERR_MISUSE, "cq: a residual add takes one matrix and no activation");
    for (int k = 0; k < n; ++k) {
        if (!ms[k] || ms[k]->st->in != ms[0]->st->in)
            return fail(CQ_ERR_MISUSE, "cq: GEMMs over matrices of different input widths");
        if (!uses_lut(ms[k]))
            return fail(CQ_ERR_UNSUPPORTED, "cq: fused products run the lut kernel, not %s", cq_kernel_name(ms[k]));
    }
    if (int e = nil_operands(n, dsts, x, rows)) return e;
    if (rows == 0 || n == 0) return CQ_OK;
    Fuse f;
    f.ngain = norm_gain;
    f.resid = resid;
    f.resid_stride = resid ? ms[0]->out : 0;
    f.act = act;
    return gemms_dev(n, ms, dsts, x, rows, static_cast<hipStream_t>(stream), &f);
}

int cq_gemms_gated_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, const float *gate, int rows,
                       const float *resid, void *stream) {
    if (n < 0 || (n > 0 && (!ms || !dsts))) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d matrices", n);
    if (rows < 0) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d rows", rows);
    if (!gate && rows > 0 && n > 0) return fail(CQ_ERR_MISUSE, "cq: gated GEMMs without a gate");
    if (resid && n != 1) return fail(CQ_ERR_MISUSE, "cq: a residual add takes one matrix");
    for (int k = 0; k < n; ++k) {
        if (!ms[k] || ms[k]->st->in != ms[0]->st->in)
            return fail(CQ_ERR_MISUSE, "cq: GEMMs over matrices of different input widths");
        if (!uses_lut(ms[k]))
            return fail(CQ_ERR_UNSUPPORTED, "cq: fused products run the lut kernel, not %s", cq_kernel_name(ms[k]));
    }
    if (int e = nil_operands(n, dsts, x, rows)) return e;
    if (rows == 0 || n == 0) return CQ_OK;
    Fuse f;
    f.xgate = gate;
    f.resid = resid;
    f.resid_stride = resid ? ms[0]->out : 0;
    return gemms_dev(n, ms, dsts, x, rows, static_cast<hipStream_t>(stream), &f);
}

int cq_gemms_append_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows,
                        const float *norm_gain, int8_t *const *kv_q, float *const *kv_s, long long q_stride,
                        long long s_stride, const int32_t *pos, int cap, const float *const *cos_t,
                        const float *const *sin_t, void *stream) {
    if (n < 0 || n > kKernargJobs || (n > 0 && (!ms || !dsts || !kv_q || !kv_s)))
        return fail(CQ_ERR_MISUSE, "cq: appending GEMMs of %d matrices (at most %d)", n, kKernargJobs);
    if (rows < 0 || cap < 0) return fail(CQ_ERR_MISUSE, "cq: appending GEMMs of %d rows into %d positions", rows, cap);
    bool any = false;
    for (int k = 0; k < n; ++k) {
        if (!ms[k] || ms[k]->st->in != ms[0]->st->in)
            return fail(CQ_ERR_MISUSE, "cq: GEMMs over matrices of different input widths");
        const CqStore &sk = *ms[k]->st, &s0 = *ms[0]->st;  // each workgroup builds its own job's tables
        if (!uses_lut(ms[k]) || !lut_fits(sk) || sk.group != s0.group || sk.width != s0.width ||
            sk.group_bytes != s0.group_bytes)
            return fail(CQ_ERR_UNSUPPORTED, "cq: appending products run one lut kernel over matrices of one geometry");
        if (!kv_q[k]) continue;
        any = true;
        if (!kv_s[k] || ms[k]->row0 % kBlockRows || ms[k]->out % kBlockRows)
            return fail(CQ_ERR_MISUSE, "cq: append of rows [%d, %d) needs scales and heads of %d rows", ms[k]->row0,
                        ms[k]->row0 + ms[k]->out, kBlockRows);
        if (cos_t && cos_t[k] && !(sin_t && sin_t[k])) return fail(CQ_ERR_MISUSE, "cq: RoPE cosines without sines");
    }
    if (any && !pos) return fail(CQ_ERR_MISUSE, "cq: append without positions");
    if (int e = nil_operands(n, dsts, x, rows)) return e;
    if (rows == 0 || n == 0) return CQ_OK;
    Fuse f;
    f.ngain = norm_gain;
    if (any) {
        f.app_q = kv_q;
        f.app_s = kv_s;
        f.app_cos = cos_t;
        f.app_sin = sin_t;
        f.app_q_stride = q_stride;
        f.app_s_stride = s_stride;
        f.app_pos = pos;
        f.app_cap = cap;
    }
    // the table and split MFMA forms append in their folds (whole 64-row
    // blocks, checked above)
    if (tab_pays(ms, n, rows)) return run_tab(ms, n, dsts, x, rows, static_cast<hipStream_t>(stream), &f);
    if (split_pays(ms, n, rows)) return run_split(ms, n, dsts, x, rows, static_cast<hipStream_t>(stream), &f);
    return run_lut(ms, n, dsts, x, rows, static_cast<hipStream_t>(stream), &f);
}

size_t cq_tables_bytes(int n, cq_matrix *const *ms, int rows) {
    if (n <= 0 || n > kKernargJobs || !ms || rows <= 0) return 0;
    for (int k = 0; k < n; ++k)
        if (!ms[k] || ms[k]->st->in != ms[0]->st->in || ms[k]->dense) return 0;
    if (!tab_pays(ms, n, rows)) return 0;
    const CqStore &s0 = *ms[0]->st;
    const int tiles = (rows + 31) / 32;
    return tab_table_bytes(s0.width, s0.groups, tiles) + tab_step_bytes(s0.groups, tiles);
}

int cq_gemm_tables_dev(const cq_matrix *m, float *dst, const float *x, const float *gate, int rows, const float *resid,
                       int n_next, cq_matrix *const *next, const float *next_gain, void *tables, size_t tables_bytes,
                       int *built, void *stream) {
    if (!built) return fail(CQ_ERR_MISUSE, "cq: a table-building GEMM without its flag");
    *built = 0;
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (rows < 0) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d rows", rows);
    if (!uses_lut(m))
        return fail(CQ_ERR_UNSUPPORTED, "cq: fused products run the lut kernel, not %s", cq_kernel_name(m));
    if (n_next < 1 || n_next > kKernargJobs || !next)
        return fail(CQ_ERR_MISUSE, "cq: tables for a product of %d matrices (1 to %d)", n_next, kKernargJobs);
    for (int k = 0; k < n_next; ++k)
        if (!next[k] || next[k]->st->in != m->out)
            return fail(CQ_ERR_MISUSE, "cq: the next product's matrices must take the %d outputs as inputs", m->out);
    if (int e = nil_operands(1, &dst, x, rows)) return e;
    if (rows == 0 || m->out == 0) return CQ_OK;
    const size_t need = cq_tables_bytes(n_next, next, rows);
    if (tables_bytes != need || (need && !tables))
        return fail(CQ_ERR_MISUSE, "cq: a table buffer of %zu bytes where the next product's tables take %zu",
                    tables_bytes, need);
    Fuse f;
    f.xgate = gate;
    f.resid = resid;
    f.resid_stride = resid ? m->out : 0;
    cq_matrix *mm = const_cast<cq_matrix *>(m);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (need == 0) return run_product(&mm, 1, &dst, x, rows, st, &f);
    const CqStore &n0 = *next[0]->st;
    const int tiles = (rows + 31) / 32;
    TabOut to;
    std::memset(&to, 0, sizeof to);
    to.tab = static_cast<int8_t *>(tables);
    to.stp = reinterpret_cast<float *>(static_cast<char *>(tables) + tab_table_bytes(n0.width, n0.groups, tiles));
    to.ngain = next_gain;
    to.in = n0.in;
    to.groups = n0.groups;
    to.bits = n0.width;
    to.tiles = tiles;
    for (int c = 0; c < 16; ++c) to.cb[c] = c < n0.ncb ? n0.cb[c] : 0.0f;
    to.cb_max = n0.cb_max;
    to.lut_step = n0.lut_step;
    return run_product(&mm, 1, &dst, x, rows, st, &f, &to, built);
}

int cq_gemms_tables_dev(int n, cq_matrix *const *ms, float *const *dsts, int rows, const float *resid, int act,
                        int8_t *const *kv_q, float *const *kv_s, long long q_stride, long long s_stride,
                        const int32_t *pos, int cap, const float *const *cos_t, const float *const *sin_t,
                        const void *tables, size_t tables_bytes, void *stream) {
    if (n < 1 || n > kKernargJobs || !ms || !dsts)
        return fail(CQ_ERR_MISUSE, "cq: GEMMs over tables of %d matrices (1 to %d)", n, kKernargJobs);
    if (rows < 0 || cap < 0) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d rows into %d positions", rows, cap);
    if (act != 0 && act != 1) return fail(CQ_ERR_MISUSE, "cq: activation %d", act);
    if (resid && (n != 1 || act != 0))
        return fail(CQ_ERR_MISUSE, "cq: a residual add takes one matrix and no activation");
    bool any = false;
    for (int k = 0; k < n; ++k) {
        if (!ms[k] || ms[k]->st->in != ms[0]->st->in)
            return fail(CQ_ERR_MISUSE, "cq: GEMMs over matrices of different input widths");
        if (!dsts[k] && rows > 0) return fail(CQ_ERR_MISUSE, "cq: GEMMs with a nil output %d", k);
        if (!kv_q || !kv_q[k]) continue;
        any = true;
        if (!kv_s || !kv_s[k] || ms[k]->row0 % kBlockRows || ms[k]->out % kBlockRows)
            return fail(CQ_ERR_MISUSE, "cq: append of rows [%d, %d) needs scales and heads of %d rows", ms[k]->row0,
                        ms[k]->row0 + ms[k]->out, kBlockRows);
        if (cos_t && cos_t[k] && !(sin_t && sin_t[k])) return fail(CQ_ERR_MISUSE, "cq: RoPE cosines without sines");
    }
    if (any && !pos) return fail(CQ_ERR_MISUSE, "cq: append without positions");
    if (rows == 0) return CQ_OK;
    const size_t need = cq_tables_bytes(n, ms, rows);
    if (need == 0)
        return fail(CQ_ERR_MISUSE, "cq: this product of %d rows does not take the table form (no tables)", rows);
    if (!tables || tables_bytes != need)
        return fail(CQ_ERR_MISUSE, "cq: a table buffer of %zu bytes where the product's tables take %zu", tables_bytes,
                    need);
    Fuse f;
    f.resid = resid;
    f.resid_stride = resid ? ms[0]->out : 0;
    f.act = act;
    if (any) {
        f.app_q = kv_q;
        f.app_s = kv_s;
        f.app_cos = cos_t;
        f.app_sin = sin_t;
        f.app_q_stride = q_stride;
        f.app_s_stride = s_stride;
        f.app_pos = pos;
        f.app_cap = cap;
    }
    return run_tab(ms, n, dsts, nullptr, rows, static_cast<hipStream_t>(stream), &f, tables);
}

int cq_gemm(const cq_matrix *m, float *dst, size_t dst_len, const float *x, size_t x_len, int rows) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    const CqStore &s = *m->st;
    // kernel.go:100-103
    if (rows < 0 || x_len != static_cast<size_t>(rows) * s.in || dst_len != static_cast<size_t>(rows) * m->out)
        return fail(CQ_ERR_MISUSE, "cq: GEMM(len %zu, len %zu, %d rows) on [%d, %d]", dst_len, x_len, rows, m->out,
                    s.in);
    if (rows == 0 || m->out == 0) return CQ_OK;
    const size_t xb = align256(x_len * 4), yb = align256(dst_len * 4);
    HIP_TRY(t_stage.ensure(xb + yb), "staging");
    char *base = static_cast<char *>(t_stage.buf);
    float *dx = reinterpret_cast<float *>(base), *dy = reinterpret_cast<float *>(base + xb);
    HIP_TRY(hipMemcpyAsync(dx, x, x_len * 4, hipMemcpyHostToDevice, t_stage.stream), "copy x");
    cq_matrix *mm = const_cast<cq_matrix *>(m);
    int rc = run_product(&mm, 1, &dy, dx, rows, t_stage.stream);
    if (rc) {
        (void)hipStreamSynchronize(t_stage.stream);
        return rc;
    }
    HIP_TRY(hipMemcpyAsync(dst, dy, dst_len * 4, hipMemcpyDeviceToHost, t_stage.stream), "copy y");
    HIP_TRY(hipStreamSynchronize(t_stage.stream), "sync");
    return CQ_OK;
}

int cq_gemms(int n, cq_matrix *const *ms, float *const *dsts, const size_t *dst_lens, const float *x, size_t x_len,
             int rows) {
    if (n < 0 || (n > 0 && (!ms || !dsts || !dst_lens))) return fail(CQ_ERR_MISUSE, "cq: GEMMs of %d matrices", n);
    // kernel.go:135-144
    for (int k = 0; k < n; ++k) {
        const cq_matrix *m = ms[k];
        if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
        if (rows < 0 || x_len != static_cast<size_t>(rows) * m->st->in ||
            dst_lens[k] != static_cast<size_t>(rows) * m->out)
            return fail(CQ_ERR_MISUSE, "cq: GEMMs(len %zu, len %zu, %d rows) on [%d, %d]", dst_lens[k], x_len, rows,
                        m->out, m->st->in);
    }
    if (rows == 0 || n == 0) return CQ_OK;
    size_t total = align256(x_len * 4);
    std::vector<size_t> off(n);
    for (int k = 0; k < n; ++k) {
        off[k] = total;
        total += align256(dst_lens[k] * 4);
    }
    HIP_TRY(t_stage.ensure(total), "staging");
    char *base = static_cast<char *>(t_stage.buf);
    float *dx = reinterpret_cast<float *>(base);
    std::vector<float *> dy(n);
    for (int k = 0; k < n; ++k) dy[k] = reinterpret_cast<float *>(base + off[k]);
    HIP_TRY(hipMemcpyAsync(dx, x, x_len * 4, hipMemcpyHostToDevice, t_stage.stream), "copy x");
    int rc = gemms_dev(n, ms, dy.data(), dx, rows, t_stage.stream);
    if (rc) {
        (void)hipStreamSynchronize(t_stage.stream);
        return rc;
    }
    for (int k = 0; k < n; ++k)
        if (dst_lens[k])
            HIP_TRY(hipMemcpyAsync(dsts[k], dy[k], dst_lens[k] * 4, hipMemcpyDeviceToHost, t_stage.stream), "copy y");
    HIP_TRY(hipStreamSynchronize(t_stage.stream), "sync");
    return CQ_OK;
}

int cq_row_dev(const cq_matrix *m, float *dst, int r, void *stream) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (r < 0 || r >= m->out) return fail(CQ_ERR_MISUSE, "cq: Row(%d) of [%d, %d]", r, m->out, m->st->in);
    RowArgs a;
    int rc = row_args(m, a);
    if (rc) return rc;
    a.dst = dst;
    a.r0 = m->row0 + r;
    a.n = 1;
    HIP_TRY(launch_rows(a, static_cast<hipStream_t>(stream)), "row launch");
    return CQ_OK;
}

int cq_row_gather_dev(const cq_matrix *m, float *dst, const int32_t *rows, int n, float scale, void *stream) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    if (n < 0) return fail(CQ_ERR_MISUSE, "cq: gather of %d rows", n);
    if (m->row0 != 0) return fail(CQ_ERR_UNSUPPORTED, "cq: row gather on a Rows view");
    RowArgs a;
    int rc = row_args(m, a);
    if (rc) return rc;
    a.dst = dst;
    a.rows = rows;
    a.n = n;
    a.scale = scale;
    HIP_TRY(launch_rows(a, static_cast<hipStream_t>(stream)), "row gather launch");
    return CQ_OK;
}

int cq_row(const cq_matrix *m, float *dst, size_t dst_len, int r) {
    if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix");
    // matrix.go:162-164
    if (r < 0 || r >= m->out || dst_len != static_cast<size_t>(m->st->in))
        return fail(CQ_ERR_MISUSE, "cq: Row(len %zu, %d) of [%d, %d]", dst_len, r, m->out, m->st->in);
    HIP_TRY(t_stage.ensure(align256(dst_len * 4)), "staging");
    float *dd = static_cast<float *>(t_stage.buf);
    int rc = cq_row_dev(m, dd, r, t_stage.stream);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(dst, dd, dst_len * 4, hipMemcpyDeviceToHost, t_stage.stream), "copy row");
    HIP_TRY(hipStreamSynchronize(t_stage.stream), "sync");
    return CQ_OK;
}

// ---- batch plans: many independent products in few launches -----------------

}  // extern "C"

struct cq_batch {
    struct Launch {
        int bits, gb, waves, grid;
        size_t lds;
        LutLaunch args;
    };
    std::vector<Launch> launches;
    std::vector<void *> dev_mem;
    std::vector<std::shared_ptr<CqStore>> keep;  // storage stays alive with the plan
    ~cq_batch() {
        for (void *p : dev_mem) (void)hipFree(p);
    }
};

extern "C" {

int cq_batch_new(int n, cq_matrix *const *ms, float *const *ys, const float *const *xs, const int *rows,
                 cq_batch **plan) {
    if (!plan || n < 0 || (n > 0 && (!ms || !ys || !xs || !rows))) return fail(CQ_ERR_MISUSE, "cq: batch of %d", n);
    *plan = nullptr;
    auto b = std::make_unique<cq_batch>();
    // Jobs by kernel geometry (bits, group bytes): one launch each.
    std::vector<std::pair<std::pair<int, int>, std::vector<int>>> classes;
    for (int k = 0; k < n; ++k) {
        const cq_matrix *m = ms[k];
        if (!m) return fail(CQ_ERR_MISUSE, "cq: nil matrix in batch");
        if (rows[k] < 0) return fail(CQ_ERR_MISUSE, "cq: batch job %d of %d rows", k, rows[k]);
        if (!uses_lut(m) || !lut_fits(*m->st))
            return fail(CQ_ERR_UNSUPPORTED, "cq: batch job %d needs the %s kernel; batches run the lut kernel", k,
                        cq_kernel_name(m));
        if (m->out == 0 || rows[k] == 0) continue;
        const std::pair<int, int> key{m->st->width, m->st->group_bytes};
        auto it = std::find_if(classes.begin(), classes.end(), [&](auto &c) { return c.first == key; });
        if (it == classes.end()) {
            classes.push_back({key, {}});
            it = classes.end() - 1;
        }
        it->second.push_back(k);
        b->keep.push_back(m->st);
    }
    for (auto &cls : classes) {
        std::vector<JobDesc> jobs;
        std::vector<WorkUnit> units;
        // Workgroups get about equal index bytes: total / (4 per CU), in whole
        // 64-row blocks (at most kLutMaxBpw), heaviest units first.
        long long bytes = 0;
        for (int k : cls.second)
            bytes += static_cast<long long>((ms[k]->row0 + ms[k]->out + 63) / 64 - ms[k]->row0 / 64) * 64 *
                     ms[k]->st->row_bytes * rows[k];
        const long long target = std::max<long long>(1, bytes / (4LL * device_info().cus));
        int bpw = 1;
        std::vector<std::pair<long long, WorkUnit>> weighted;
        for (int k : cls.second) {
            JobDesc j;
            fill_job(j, ms[k], xs[k], ys[k], rows[k]);
            const long long blk_bytes = 64LL * ms[k]->st->row_bytes;
            const int b = balanced_blocks(
                j.nblk, static_cast<int>(std::min<long long>(kLutMaxBpw, std::max<long long>(1, target / blk_bytes))));
            bpw = std::max(bpw, b);
            const int ji = static_cast<int>(jobs.size());
            jobs.push_back(j);
            for (int act = 0; act < rows[k]; ++act)
                for (int blk = 0; blk < j.nblk; blk += b) {
                    const int nb = std::min(b, j.nblk - blk);
                    weighted.push_back({nb * blk_bytes, WorkUnit{ji, blk, nb, act}});
                }
        }
        std::stable_sort(weighted.begin(), weighted.end(),
                         [](const auto &p, const auto &q) { return p.first > q.first; });
        for (auto &wu : weighted) units.push_back(wu.second);
        int groups_max = 0;
        for (auto &j : jobs) groups_max = std::max(groups_max, j.groups);
        void *dj = nullptr, *du = nullptr;
        HIP_TRY(hipMalloc(&dj, align256(jobs.size() * sizeof(JobDesc))), "hipMalloc batch jobs");
        b->dev_mem.push_back(dj);
        HIP_TRY(hipMalloc(&du, align256(units.size() * sizeof(WorkUnit))), "hipMalloc batch units");
        b->dev_mem.push_back(du);
        HIP_TRY(hipMemcpy(dj, jobs.data(), jobs.size() * sizeof(JobDesc), hipMemcpyHostToDevice), "upload jobs");
        HIP_TRY(hipMemcpy(du, units.data(), units.size() * sizeof(WorkUnit), hipMemcpyHostToDevice), "upload units");
        cq_batch::Launch L;
        std::memset(&L.args, 0, sizeof L.args);
        L.bits = cls.first.first;
        L.gb = cls.first.second;
        L.waves = kLutWaves;
        L.args.djobs = static_cast<const JobDesc *>(dj);
        L.args.dunits = static_cast<const WorkUnit *>(du);
        L.args.tb = kLutTile;
        L.args.gc = lut_chunk(groups_max);
        L.args.bpw_max = bpw;
        L.lds = lut_lds_bytes(L.bits, L.gb, L.args.gc, kLutTile, bpw);
        L.grid = static_cast<int>(units.size());
        b->launches.push_back(L);
    }
    for (int k = 0; k < n; ++k) ms[k]->st->prepared.store(true);
    *plan = b.release();
    return CQ_OK;
}

int cq_batch_run(const cq_batch *plan, void *stream) {
    if (!plan) return fail(CQ_ERR_MISUSE, "cq: nil batch");
    for (const auto &L : plan->launches)
        for (int g0 = 0; g0 < L.grid; g0 += 1 << 30) {
            LutLaunch a = L.args;
            a.dunits += g0;
            HIP_TRY(launch_lut(a, L.bits, L.gb, L.waves, std::min(L.grid - g0, 1 << 30), 1, L.lds,
                               static_cast<hipStream_t>(stream)),
                    "batch launch");
        }
    return CQ_OK;
}

int cq_batch_launches(const cq_batch *plan) { return plan ? static_cast<int>(plan->launches.size()) : 0; }

void cq_batch_free(cq_batch *plan) { delete plan; }

// ---- int8 KV -----------------------------------------------------------------

int kv_quantize_rows_dev(int8_t *q, float *s, const float *x, int rows, int cols, int width, void *stream) {
    // NewInt8Rows / Append checks (int8.go:107-128)
    if (width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 rows of %d in chunks of %d", cols, width);
    if (rows < 0) return fail(CQ_ERR_MISUSE, "needle: %d rows", rows);
    const long long chunks = static_cast<long long>(rows) * (cols / width);
    HIP_TRY(launch_quantize_rows(q, s, x, chunks, width, static_cast<hipStream_t>(stream)), "quantize launch");
    return CQ_OK;
}

int kv_reorder_dev(int8_t *q, float *s, int8_t *tmp_q, float *tmp_s, const int32_t *parent, const int32_t *len,
                   int streams, int cap, int cols, int width, void *stream) {
    if (width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 rows of %d in chunks of %d", cols, width);
    if (streams < 0 || cap < 0) return fail(CQ_ERR_MISUSE, "needle: %d streams of %d rows", streams, cap);
    if (streams == 0 || cap == 0) return CQ_OK;
    if (!q || !s || !tmp_q || !tmp_s || !parent || !len || tmp_q == q || tmp_s == s)
        return fail(CQ_ERR_MISUSE, "needle: reorder needs caches, distinct temporaries, parents and lengths");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const int sb = (cols / width) * static_cast<int>(sizeof(float));
    // through the temporaries: a stream may be another's parent
    HIP_TRY(launch_gather_rows(tmp_q, q, parent, len, streams, cap, cols, st), "reorder gather");
    HIP_TRY(launch_gather_rows(tmp_s, s, parent, len, streams, cap, sb, st), "reorder gather");
    HIP_TRY(launch_gather_rows(q, tmp_q, nullptr, len, streams, cap, cols, st), "reorder copy back");
    HIP_TRY(launch_gather_rows(s, tmp_s, nullptr, len, streams, cap, sb, st), "reorder copy back");
    return CQ_OK;
}

// ---- the allocation-free reorder ------------------------------------------
//
// kv_reorder_noalloc_dev keeps kv_reorder_dev's temporaries in `scratch`, a
// file-scope device array of kScratchBytes that every GPU the library runs
// on holds until the process ends. Host code never uses the array's name as
// an address (on the host it is only a stand-in for the symbol): the device
// address comes from hipGetSymbolAddress, once per device, with that device
// current, and is kept per device. Every call on one GPU shares that GPU's
// array, so calls that overlap on one GPU (different streams, or threads
// without ordering) race; the reorder needs nothing in it cleared.
}  // extern "C"

// 16 MiB: a 256-stream reorder of 64 rows of 512 codes (8.5 MiB with its
// scales) fits; the paged self caches' forks share pages and need none.
constexpr size_t kScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char *g_scratch_ptr[kMaxDevices];  // per device: the array's device address

int scratch_of_current_device(unsigned char **out) {
    int dev = -1;
    HIP_TRY(hipGetDevice(&dev), "current device");
    if (dev < 0 || dev >= kMaxDevices) return fail(CQ_ERR_DEVICE, "needle: device %d has no scratch slot", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "scratch address");
        g_scratch_ptr[dev] = static_cast<unsigned char *>(p);
    }
    *out = g_scratch_ptr[dev];
    return CQ_OK;
}
}  // namespace

extern "C" {

int kv_reorder_noalloc_dev(int8_t *q, float *s, const int32_t *parent, const int32_t *len, int streams, int cap,
                           int cols, int width, void *stream) {
    if (width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 rows of %d in chunks of %d", cols, width);
    if (streams < 0 || cap < 0) return fail(CQ_ERR_MISUSE, "needle: %d streams of %d rows", streams, cap);
    if (streams == 0 || cap == 0) return CQ_OK;
    if (!q || !s || !parent || !len) return fail(CQ_ERR_MISUSE, "needle: reorder needs caches, parents and lengths");
    const int sb = (cols / width) * static_cast<int>(sizeof(float));
    const size_t rows = static_cast<size_t>(streams) * static_cast<size_t>(cap);
    const size_t qbytes = align256(rows * static_cast<size_t>(cols)), need = qbytes + rows * static_cast<size_t>(sb);
    if (need > kScratchBytes)
        return fail(CQ_ERR_MISUSE,
                    "needle: a reorder of %d streams of %d rows of %d codes needs %zu bytes of temporaries; the "
                    "allocation-free form holds %zu (use kv_reorder_dev with temporaries of your own)",
                    streams, cap, cols, need, kScratchBytes);
    unsigned char *base = nullptr;
    if (int e = scratch_of_current_device(&base)) return e;
    int8_t *tmp_q = reinterpret_cast<int8_t *>(base);
    float *tmp_s = reinterpret_cast<float *>(base + qbytes);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    HIP_TRY(launch_gather_rows(tmp_q, q, parent, len, streams, cap, cols, st), "reorder gather");
    HIP_TRY(launch_gather_rows(tmp_s, s, parent, len, streams, cap, sb, st), "reorder gather");
    HIP_TRY(launch_gather_rows(q, tmp_q, nullptr, len, streams, cap, cols, st), "reorder copy back");
    HIP_TRY(launch_gather_rows(s, tmp_s, nullptr, len, streams, cap, sb, st), "reorder copy back");
    return CQ_OK;
}

int nd_fake_quant_dev(float *dst, const float *x, long long rows, int cols, int width, void *stream) {
    if (width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 rows of %d in chunks of %d", cols, width);
    if (rows < 0) return fail(CQ_ERR_MISUSE, "needle: %lld rows", rows);
    HIP_TRY(launch_fake_quant(dst, x, rows * (cols / width), width, static_cast<hipStream_t>(stream)),
            "fake quant launch");
    return CQ_OK;
}

int kv_quantize_rows(int8_t *q, float *s, const float *x, int rows, int cols, int width) {
    if (width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 rows of %d in chunks of %d", cols, width);
    if (rows < 0) return fail(CQ_ERR_MISUSE, "needle: %d rows", rows);
    const size_t n = static_cast<size_t>(rows) * cols, chunks = static_cast<size_t>(rows) * (cols / width);
    if (n == 0) return CQ_OK;
    const size_t xb = align256(n * 4), qb = align256(n), sb = align256(chunks * 4);
    HIP_TRY(t_stage.ensure(xb + qb + sb), "staging");
    char *base = static_cast<char *>(t_stage.buf);
    float *dx = reinterpret_cast<float *>(base);
    int8_t *dq = reinterpret_cast<int8_t *>(base + xb);
    float *ds = reinterpret_cast<float *>(base + xb + qb);
    HIP_TRY(hipMemcpyAsync(dx, x, n * 4, hipMemcpyHostToDevice, t_stage.stream), "copy x");
    int rc = kv_quantize_rows_dev(dq, ds, dx, rows, cols, width, t_stage.stream);
    if (rc) return rc;
    HIP_TRY(hipMemcpyAsync(q, dq, n, hipMemcpyDeviceToHost, t_stage.stream), "copy q");
    HIP_TRY(hipMemcpyAsync(s, ds, chunks * 4, hipMemcpyDeviceToHost, t_stage.stream), "copy s");
    HIP_TRY(hipStreamSynchronize(t_stage.stream), "sync");
    return CQ_OK;
}

static int attend_impl(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                       const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                       int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans, int nk_max,
                       float scale, int quant_q, int batch, const float *rope_cos, const float *rope_sin,
                       const int32_t *qpos, const int32_t *kv_index, int kv_streams, void *stream,
                       const int32_t *pages = nullptr, int page_stride = 0, int page_rows = 0, int pool_pages = 0) {
    if (rope_cos && (!rope_sin || !qpos || qk % 2 != 0))
        return fail(CQ_ERR_MISUSE, "needle: RoPE of query heads of %d", qk);
    if (kv_index && kv_streams < 0) return fail(CQ_ERR_MISUSE, "needle: %d shared caches", kv_streams);
    if (static_cast<long long>(t) * heads * batch > 0 && (!out || !q || !kq || !ks || !vq || !vs || !spans))
        return fail(CQ_ERR_MISUSE, "needle: int8 attention with a nil operand");
    if (qk <= 0 || vd <= 0 || k_cols % qk != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 keys of %d in chunks of %d", k_cols, qk);
    const int kv_heads = k_cols / qk;
    if (heads <= 0 || heads % kv_heads != 0 || v_cols != kv_heads * vd)
        return fail(CQ_ERR_MISUSE, "needle: %d heads over %d KV heads (values %d of %d)", heads, kv_heads, v_cols, vd);
    if (qk > 256 || qk % 4 != 0 || k_cols % 4 != 0 || vd > 192)
        return fail(CQ_ERR_UNSUPPORTED, "needle: int8 attention with head widths %d and %d", qk, vd);
    if (t < 0 || batch < 0 || nk_max < 0) return fail(CQ_ERR_MISUSE, "needle: bad attention sizes");
    if (nk_max > 8192) return fail(CQ_ERR_UNSUPPORTED, "needle: %d keys exceed LDS", nk_max);
    if (out_stride == 0) out_stride = static_cast<long long>(t) * heads * vd;  // dense streams
    if (q_stride == 0) q_stride = static_cast<long long>(t) * heads * qk;
    // Value codes in LDS: all of a stream's rows at once (their loads overlap
    // the logits) when the launch has few workgroups and they fit in 96 KiB;
    // else two buffers of 256 rows, for more workgroups per CU.
    const long long wgs = static_cast<long long>(heads) * t * batch;
    const int fit = static_cast<int>(96 * 1024 / vd);
    const int vchunk = (wgs <= 2LL * device_info().cus && nk_max <= fit) ? std::max(1, nk_max) : std::min(256, fit / 2);
    const int resident = wgs <= 2LL * device_info().cus ? 1 : 0;
    int page_shift = 0;
    if (pages) {
        if (kv_index) return fail(CQ_ERR_MISUSE, "needle: paged caches with a shared-cache index");
        if (page_rows <= 0 || (page_rows & (page_rows - 1)) != 0 ||
            static_cast<long long>(page_stride) * page_rows < nk_max || pool_pages <= 0)
            return fail(CQ_ERR_MISUSE, "needle: %d pages of %d rows for %d keys (pool %d)", page_stride, page_rows,
                        nk_max, pool_pages);
        while ((1 << page_shift) < page_rows) ++page_shift;
        if ((nk_max + page_rows - 1) / page_rows > kAttendMaxPages)
            return fail(CQ_ERR_UNSUPPORTED, "needle: %d keys in pages of %d rows", nk_max, page_rows);
        kv_stride = s_stride = 0;  // the page table gives every row
    }
    AttendArgs a{out, out_stride, q, q_stride, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd,
                 kv_stride, s_stride, spans, nk_max, vchunk, resident, scale, quant_q, batch,
                 rope_cos, rope_sin, qpos, kv_index, kv_streams, pages, page_stride, page_shift, pool_pages};
    HIP_TRY(launch_attend_int8(a, static_cast<hipStream_t>(stream)), "attend launch");
    return CQ_OK;
}

int kv_attend_int8_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                       const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                       int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans, int nk_max,
                       float scale, int quant_q, int batch, void *stream) {
    return attend_impl(out, out_stride, q, q_stride, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, kv_stride,
                       s_stride, spans, nk_max, scale, quant_q, batch, nullptr, nullptr, nullptr, nullptr, 0, stream);
}

int kv_attend_int8_shared_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                              const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                              int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans,
                              int nk_max, float scale, int quant_q, int batch, const int32_t *kv_index, int kv_streams,
                              void *stream) {
    if (!kv_index && static_cast<long long>(t) * heads * batch > 0)
        return fail(CQ_ERR_MISUSE, "needle: shared caches without an index");
    return attend_impl(out, out_stride, q, q_stride, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, kv_stride,
                       s_stride, spans, nk_max, scale, quant_q, batch, nullptr, nullptr, nullptr, kv_index, kv_streams,
                       stream);
}

int kv_attend_int8_rope_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                            const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                            int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans,
                            int nk_max, float scale, int quant_q, int batch, const float *cos_t, const float *sin_t,
                            const int32_t *qpos, void *stream) {
    if (!cos_t) return fail(CQ_ERR_MISUSE, "needle: RoPE tables missing");
    return attend_impl(out, out_stride, q, q_stride, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, kv_stride,
                       s_stride, spans, nk_max, scale, quant_q, batch, cos_t, sin_t, qpos, nullptr, 0, stream);
}

int kv_attend_int8_paged_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                             const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                             int v_cols, int vd, const int32_t *spans, int nk_max, float scale, int quant_q, int batch,
                             const float *cos_t, const float *sin_t, const int32_t *qpos, const int32_t *pages,
                             int page_stride, int page_rows, int pool_pages, void *stream) {
    if (!pages && static_cast<long long>(t) * heads * batch > 0)
        return fail(CQ_ERR_MISUSE, "needle: paged caches without a page table");
    if (cos_t && (!sin_t || !qpos)) return fail(CQ_ERR_MISUSE, "needle: RoPE tables missing");
    return attend_impl(out, out_stride, q, q_stride, t, heads, kq, ks, k_cols, qk, vq, vs, v_cols, vd, 0, 0, spans,
                       nk_max, scale, quant_q, batch, cos_t, sin_t, qpos, nullptr, 0, stream, pages, page_stride,
                       page_rows, pool_pages);
}

int nd_qkv_prep_dev(float *q, const float *k, const float *v, int batch, int dim, float *hist, const float *taps_w,
                    int taps, const float *q_gain, const float *k_gain, const float *cos_t, const float *sin_t,
                    int positions, const int32_t *pos, int cap, int8_t *kq, float *ks, int8_t *vq, float *vs,
                    const int32_t *pages, int page_stride, int page_rows, int pool_pages, void *stream) {
    if (batch < 0 || dim <= 0 || dim % 64 != 0 || dim > 1024 || taps < 0 || cap < 0)
        return fail(CQ_ERR_MISUSE, "needle: q/k/v of %d rows of %d with %d taps", batch, dim, taps);
    if (batch == 0) return CQ_OK;
    if (!q || !k || !v || !pos || !kq || !ks || !vq || !vs || !pages || (taps > 0 && !taps_w) ||
        (taps > 1 && !hist) || (cos_t && !sin_t))
        return fail(CQ_ERR_MISUSE, "needle: q/k/v preparation with a nil operand");
    if (page_rows <= 0 || (page_rows & (page_rows - 1)) != 0 || static_cast<long long>(page_stride) * page_rows < cap ||
        pool_pages <= 0)
        return fail(CQ_ERR_MISUSE, "needle: %d pages of %d rows for %d positions (pool %d)", page_stride, page_rows,
                    cap, pool_pages);
    int shift = 0;
    while ((1 << shift) < page_rows) ++shift;
    PrepArgs a{q, k, v, hist, taps_w, taps, q_gain, k_gain, cos_t, sin_t, positions, pos, cap, kq, vq, ks, vs,
               pages, page_stride, shift, pool_pages, dim};
    HIP_TRY(launch_qkv_prep(a, batch, static_cast<hipStream_t>(stream)), "q/k/v preparation launch");
    return CQ_OK;
}

int nd_norm_scaled_add_dev(float *h, const float *resid, const float *y, const float *gain, float scale, int rows,
                           int dim, void *stream) {
    if (rows < 0 || !row_kernel_dim(dim))
        return fail(CQ_ERR_MISUSE, "needle: post norm of %d rows of %d (a multiple of 256 up to 4096)", rows, dim);
    if (rows > 0 && (!h || !y || !gain)) return fail(CQ_ERR_MISUSE, "needle: post norm with a nil operand");
    HIP_TRY(launch_norm_scaled_add(h, resid ? resid : h, y, gain, scale, rows, dim, static_cast<hipStream_t>(stream)),
            "post norm launch");
    return CQ_OK;
}

int nd_rms_unit_quant_dev(float *dst, const float *x, int rows, int dim, void *stream) {
    if (rows < 0 || !row_kernel_dim(dim))
        return fail(CQ_ERR_MISUSE, "needle: RMSUnit of %d rows of %d (a multiple of 256 up to 4096)", rows, dim);
    if (rows > 0 && (!dst || !x)) return fail(CQ_ERR_MISUSE, "needle: RMSUnit with a nil operand");
    HIP_TRY(launch_rms_unit_row(dst, x, rows, dim, 1, static_cast<hipStream_t>(stream)), "RMSUnit launch");
    return CQ_OK;
}

int nd_expand_lanes_dev(float *stream_rows, const float *x, int rows, int lanes, int dim, void *stream) {
    if (rows < 0 || lanes <= 0 || dim <= 0) return fail(CQ_ERR_MISUSE, "needle: %d rows of %d lanes x %d", rows, lanes, dim);
    HIP_TRY(launch_expand_lanes(stream_rows, x, rows, lanes, dim, static_cast<hipStream_t>(stream)), "lanes launch");
    return CQ_OK;
}

int nd_collapse_lanes_dev(float *x, const float *stream_rows, int rows, int lanes, int dim, void *stream) {
    if (rows < 0 || lanes <= 0 || dim <= 0) return fail(CQ_ERR_MISUSE, "needle: %d rows of %d lanes x %d", rows, lanes, dim);
    HIP_TRY(launch_collapse_lanes(x, stream_rows, rows, lanes, dim, static_cast<hipStream_t>(stream)), "lanes launch");
    return CQ_OK;
}

int kv_page_copy_dev(int8_t *q, float *s, const int32_t *src, const int32_t *dst, int n, int page_rows, int cols,
                     int width, int pool_pages, void *stream) {
    if (n < 0 || page_rows <= 0 || cols <= 0 || width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: %d pages of %d rows of %d in heads of %d", n, page_rows, cols, width);
    if (n > 0 && (!q || !s || !src || !dst)) return fail(CQ_ERR_MISUSE, "needle: page copy with a nil operand");
    HIP_TRY(launch_page_copy(q, s, src, dst, n, page_rows, cols, cols / width, pool_pages,
                             static_cast<hipStream_t>(stream)),
            "page copy launch");
    return CQ_OK;
}

int nd_gather_rows_dev(float *dst, const float *src, const int32_t *idx, int rows, long long width, void *stream) {
    if (rows < 0 || width < 0) return fail(CQ_ERR_MISUSE, "needle: gather of %d rows of %lld", rows, width);
    if (rows > 0 && width > 0 && (!dst || !src)) return fail(CQ_ERR_MISUSE, "needle: gather with a nil operand");
    HIP_TRY(launch_gather_float_rows(dst, src, idx, rows, width, static_cast<hipStream_t>(stream)), "gather launch");
    return CQ_OK;
}

// ---- decode-step float blocks -------------------------------------------------

int nd_zcrmsnorm_dev(float *dst, const float *x, const float *gain, int rows, int dim, void *stream) {
    if (rows < 0 || dim <= 0) return fail(CQ_ERR_MISUSE, "needle: ZCRMSNorm of %d rows of %d", rows, dim);
    HIP_TRY(launch_zc_rmsnorm(dst, x, gain, rows, dim, static_cast<hipStream_t>(stream)), "norm launch");
    return CQ_OK;
}

int nd_rope_dev(float *x, int rows, int heads, int head_dim, const float *cos_t, const float *sin_t, int positions,
                const int32_t *pos, int rows_per_pos, void *stream) {
    if (rows < 0 || heads <= 0 || head_dim <= 0 || head_dim % 2 != 0 || rows_per_pos <= 0 || positions < 0)
        return fail(CQ_ERR_MISUSE, "needle: RoPE of %d rows, %d heads of %d", rows, heads, head_dim);
    if (rows > 0 && (!x || !cos_t || !sin_t || !pos)) return fail(CQ_ERR_MISUSE, "needle: RoPE with a nil operand");
    HIP_TRY(launch_rope(x, rows, heads, head_dim, cos_t, sin_t, positions, pos, rows_per_pos,
                        static_cast<hipStream_t>(stream)),
            "rope launch");
    return CQ_OK;
}

int nd_argmax_dev(int32_t *out, const float *v, int rows, int n, void *stream) {
    if (rows < 0 || n <= 0) return fail(CQ_ERR_MISUSE, "decoder: argmax of %d rows of %d", rows, n);
    if (rows > 0 && (!out || !v)) return fail(CQ_ERR_MISUSE, "decoder: argmax with a nil operand");
    HIP_TRY(launch_argmax(out, v, rows, n, nullptr, nullptr, 0, nullptr, 0, static_cast<hipStream_t>(stream)),
            "argmax launch");
    return CQ_OK;
}

int nd_argmax_advance_dev(int32_t *out, const float *v, int rows, int n, int32_t *pos, int32_t *span_hi,
                          int span_stride, void *stream) {
    if (rows < 0 || n <= 0) return fail(CQ_ERR_MISUSE, "decoder: argmax of %d rows of %d", rows, n);
    if (rows > 0 && (!out || !v || !pos || !span_hi))
        return fail(CQ_ERR_MISUSE, "decoder: argmax with a nil operand");
    HIP_TRY(launch_argmax(out, v, rows, n, pos, span_hi, span_stride, nullptr, 0, static_cast<hipStream_t>(stream)),
            "argmax launch");
    return CQ_OK;
}

int nd_argmax_advance_eos_dev(int32_t *out, const float *v, int rows, int n, int32_t *pos, int32_t *span_hi,
                              int span_stride, int32_t *done, int eos, void *stream) {
    if (rows < 0 || n <= 0) return fail(CQ_ERR_MISUSE, "decoder: argmax of %d rows of %d", rows, n);
    if (rows > 0 && (!out || !v || !pos || !span_hi || !done))
        return fail(CQ_ERR_MISUSE, "decoder: argmax with a nil operand");
    if (eos < 0 || eos >= n) return fail(CQ_ERR_MISUSE, "decoder: stop token %d outside a vocabulary of %d", eos, n);
    HIP_TRY(launch_argmax(out, v, rows, n, pos, span_hi, span_stride, done, eos, static_cast<hipStream_t>(stream)),
            "argmax launch");
    return CQ_OK;
}

int nd_silu_dev(float *x, long long n, void *stream) {
    if (n < 0) return fail(CQ_ERR_MISUSE, "needle: SiLU of %lld values", n);
    HIP_TRY(launch_silu(x, n, static_cast<hipStream_t>(stream)), "silu launch");
    return CQ_OK;
}

int nd_add_dev(float *x, const float *y, long long n, void *stream) {
    if (n < 0) return fail(CQ_ERR_MISUSE, "needle: add of %lld values", n);
    HIP_TRY(launch_add(x, y, n, static_cast<hipStream_t>(stream)), "add launch");
    return CQ_OK;
}

int nd_hadamard_mlp_dev(float *out, const float *x, int rows, int dim, int na, int nb, int rank,
                        const float *const *vecs, const float *const *factors, const float *cond_v,
                        const float *cond_u, const int32_t *p1, const int32_t *p2, void *stream) {
    if (rows < 0 || !hadamard_shape_ok(na, nb, dim, rank))
        return fail(CQ_ERR_MISUSE, "needle: HadamardMLP of %d rows, width %d in %d x %d blocks, rank %d", rows, dim, na,
                    nb, rank);
    if (rows == 0) return CQ_OK;
    if (!out || !x || !vecs || !factors || !cond_v || !cond_u || !p1 || !p2)
        return fail(CQ_ERR_MISUSE, "needle: HadamardMLP with a missing array");
    for (int k = 0; k < 5; ++k)
        if (!vecs[k]) return fail(CQ_ERR_MISUSE, "needle: HadamardMLP without vector %d", k);
    for (int k = 0; k < 6; ++k)
        if (!factors[k]) return fail(CQ_ERR_MISUSE, "needle: HadamardMLP without factor %d", k);
    HadaArgs h;
    h.out = out;
    h.x = x;
    h.dim = dim;
    h.na = na;
    h.nb = nb;
    h.rank = rank;
    h.d1 = vecs[0];
    h.d2 = vecs[1];
    h.b2 = vecs[2];
    h.d3 = vecs[3];
    h.d4 = vecs[4];
    h.w1a = factors[0];
    h.w1b = factors[1];
    h.w2a = factors[2];
    h.w2b = factors[3];
    h.w3a = factors[4];
    h.w3b = factors[5];
    h.cond_v = cond_v;
    h.cond_u = cond_u;
    h.p1 = p1;
    h.p2 = p2;
    HIP_TRY(launch_hadamard_mlp(h, rows, static_cast<hipStream_t>(stream)), "HadamardMLP launch");
    return CQ_OK;
}

int nd_rms_unit_dev(float *dst, const float *x, int rows, int dim, void *stream) {
    if (rows < 0 || dim <= 0) return fail(CQ_ERR_MISUSE, "needle: RMSUnit of %d rows of %d", rows, dim);
    if (row_kernel_dim(dim))  // 256 threads a row, the squares' chains read ahead from LDS
        HIP_TRY(launch_rms_unit_row(dst, x, rows, dim, 0, static_cast<hipStream_t>(stream)), "RMSUnit launch");
    else
        HIP_TRY(launch_rms_unit(dst, x, rows, dim, static_cast<hipStream_t>(stream)), "RMSUnit launch");
    return CQ_OK;
}

int nd_mhc_heads_dev(float *h_pre, float *h_post, float *h_res, float *u, const float *pre_logits,
                     const float *post_logits, const float *res_logits, const float *stream_rows, int rows, int lanes,
                     int dim, const float *affine, void *stream) {
    if (rows < 0 || !mhc_shape_ok(lanes, dim))
        return fail(CQ_ERR_MISUSE, "needle: mHC heads of %d rows, %d lanes of %d", rows, lanes, dim);
    if (rows == 0) return CQ_OK;
    MhcArgs m;
    std::memset(&m, 0, sizeof m);
    m.h_pre = h_pre;
    m.h_post = h_post;
    m.h_res = h_res;
    m.u = u;
    m.pre_logits = pre_logits;
    m.post_logits = post_logits;
    m.res_logits = res_logits;
    m.stream = stream_rows;
    m.affine = affine;
    m.lanes = lanes;
    m.dim = dim;
    HIP_TRY(launch_mhc_heads(m, rows, static_cast<hipStream_t>(stream)), "mHC heads launch");
    return CQ_OK;
}

int nd_mhc_heads_stacked_dev(float *h_pre, float *h_post, float *h_res, float *u, const float *logits,
                             const float *stream_rows, int rows, int lanes, int dim, const float *affine, void *stream) {
    if (rows < 0 || !mhc_shape_ok(lanes, dim))
        return fail(CQ_ERR_MISUSE, "needle: mHC heads of %d rows, %d lanes of %d", rows, lanes, dim);
    if (rows == 0) return CQ_OK;
    MhcArgs m;
    std::memset(&m, 0, sizeof m);
    m.h_pre = h_pre;
    m.h_post = h_post;
    m.h_res = h_res;
    m.u = u;
    m.pre_logits = logits;
    m.post_logits = logits + lanes;
    m.res_logits = logits + 2 * lanes;
    m.logit_stride = 2 * lanes + lanes * lanes;
    m.stream = stream_rows;
    m.affine = affine;
    m.lanes = lanes;
    m.dim = dim;
    HIP_TRY(launch_mhc_heads(m, rows, static_cast<hipStream_t>(stream)), "mHC heads launch");
    return CQ_OK;
}

int nd_mhc_mix_dev(float *out, const float *stream_rows, const float *h_res, const float *h_post,
                   const float *block_out, const float *u, int rows, int lanes, int dim, void *stream) {
    if (rows < 0 || !mhc_shape_ok(lanes, dim))
        return fail(CQ_ERR_MISUSE, "needle: mHC mix of %d rows, %d lanes of %d", rows, lanes, dim);
    if (rows == 0) return CQ_OK;
    if (out == stream_rows) return fail(CQ_ERR_MISUSE, "needle: mHC mix in place");
    MhcArgs m;
    std::memset(&m, 0, sizeof m);
    m.out = out;
    m.stream = stream_rows;
    m.h_res = const_cast<float *>(h_res);
    m.h_post = const_cast<float *>(h_post);
    m.block_out = block_out;
    m.u = const_cast<float *>(u);
    m.lanes = lanes;
    m.dim = dim;
    HIP_TRY(launch_mhc_mix(m, rows, static_cast<hipStream_t>(stream)), "mHC mix launch");
    return CQ_OK;
}

int nd_sigmoid_gate_dev(float *out, float *gate, long long n, void *stream) {
    if (n < 0) return fail(CQ_ERR_MISUSE, "needle: gate of %lld values", n);
    HIP_TRY(launch_sigmoid_gate(out, gate, n, static_cast<hipStream_t>(stream)), "gate launch");
    return CQ_OK;
}

static int append_impl(int8_t *q, float *s, const float *x, int batch, int cols, int width, long long q_stride,
                       long long s_stride, const int32_t *pos, int cap, const float *cos_t, const float *sin_t,
                       void *stream) {
    if (width <= 0 || cols % width != 0)
        return fail(CQ_ERR_MISUSE, "needle: int8 rows of %d in chunks of %d", cols, width);
    if (batch < 0 || cap < 0) return fail(CQ_ERR_MISUSE, "needle: append of %d streams", batch);
    if (width > 256) return fail(CQ_ERR_UNSUPPORTED, "needle: append in chunks of %d (at most 256)", width);
    if (cos_t && (!sin_t || width % 2 != 0)) return fail(CQ_ERR_MISUSE, "needle: RoPE of heads of %d", width);
    if (batch > 0 && cols > 0 && (!q || !s || !x || !pos))
        return fail(CQ_ERR_MISUSE, "needle: append with a nil operand");
    HIP_TRY(launch_append(q, s, x, batch, cols, width, q_stride, s_stride, pos, cap, cos_t, sin_t,
                          static_cast<hipStream_t>(stream)),
            "append launch");
    return CQ_OK;
}

int kv_append_dev(int8_t *q, float *s, const float *x, int batch, int cols, int width, long long q_stride,
                  long long s_stride, const int32_t *pos, int cap, void *stream) {
    return append_impl(q, s, x, batch, cols, width, q_stride, s_stride, pos, cap, nullptr, nullptr, stream);
}

int kv_append_rope_dev(int8_t *q, float *s, const float *x, int batch, int cols, int width, long long q_stride,
                       long long s_stride, const int32_t *pos, int cap, const float *cos_t, const float *sin_t,
                       void *stream) {
    if (!cos_t) return fail(CQ_ERR_MISUSE, "needle: RoPE tables missing");
    return append_impl(q, s, x, batch, cols, width, q_stride, s_stride, pos, cap, cos_t, sin_t, stream);
}

}  // extern "C"
