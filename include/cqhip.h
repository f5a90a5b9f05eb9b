/*
 * libcqhip: go-whistle's CQ quantized-matrix path and int8 KV numerics on
 * AMD Instinct MI355X (gfx950), behind a plain C ABI.
 *
 * Each entry point replaces one method of the reference's Go API (cited as
 * file:line in the go-whistle repository); a Go caller binds them through
 * cgo (the stub a maintainer would add is in INTEGRATION.md). Host-slice
 * entry points copy their operands to and from the device within the call,
 * as cgo requires of Go memory; the _dev entry points take device pointers
 * and a HIP stream for device-resident pipelines.
 *
 * Errors: every call returns CQ_OK or a status; cq_last_error() returns the
 * failing call's message on the calling thread. Construction errors carry
 * the reference's "cq: ..." text (the Go API returns them as error values);
 * misuse that the Go API answers with a panic (lengths that do not match
 * the shape, rows out of range) returns CQ_ERR_MISUSE.
 *
 * Threads: matrices are immutable after construction and safe for
 * concurrent use from any thread (internal/cq/matrix.go:22-24). Host-slice
 * calls run on a per-thread stream with per-thread staging buffers.
 *
 * Workspaces: the table and split forms of a batched product keep tables
 * or float terms in device memory between their two launches. They lease
 * it from one pool per process for the length of the call and return it
 * with an event behind their launches; a workspace is reused at once on the
 * stream that last used it, on another stream only once that work has
 * completed. Products queued at the same time on several streams, from one
 * thread or many, therefore never share one. A product queued while its
 * stream is captured into a graph gets a workspace that only its capture
 * sequence uses and that is held until the process ends (the graph replays
 * it at that address); such a first product of a shape may itself be
 * captured. cq_workspace_held and cq_workspace_trim report and release the
 * pool's memory.
 */
#ifndef CQHIP_H
#define CQHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    CQ_OK = 0,
    CQ_ERR_ARG = 1,         /* construction rejected: the Go API's error result */
    CQ_ERR_MISUSE = 2,      /* shape misuse: the Go API panics */
    CQ_ERR_DEVICE = 3,      /* HIP runtime failure or no device */
    CQ_ERR_UNSUPPORTED = 4, /* a geometry this library does not run */
};

/* Message of the last failing call on this thread ("" if none). */
const char *cq_last_error(void);

/* Library version string and the device it runs on (cf. `whistle doctor`,
 * cmd/whistle/doctor.go:349-370, which names the active kernels). */
const char *cq_version(void);
int cq_device_info(char *buf, size_t len);

typedef struct cq_matrix cq_matrix;

/* cq.New (internal/cq/matrix.go:46-55) when gather == 0, cq.NewGather
 * (matrix.go:60-96) when gather != 0: validates the packed form of
 * cact.Packed (internal/cact/packed.go:18-29) with the reference's checks and
 * messages, widens nothing on the host, and uploads the index and FP16 norms
 * to the device in the product layout. No host pointer is kept. */
int cq_new(int out, int in, int group, int bits, int width, const float *codebook, size_t codebook_len,
           const uint8_t *index, size_t index_len, const uint8_t *norms_fp16, size_t norms_len, int gather,
           cq_matrix **m);

/* Releases a matrix or a view; the storage goes with the last of them (the
 * Go shim calls it from a runtime.AddCleanup, as *cq.Matrix has no Close). */
void cq_free(cq_matrix *m);

int cq_out(const cq_matrix *m);  /* Matrix.Out  (matrix.go:99) */
int cq_in(const cq_matrix *m);   /* Matrix.In   (matrix.go:102) */
int cq_bits(const cq_matrix *m); /* Matrix.Bits (matrix.go:105) */
/* Matrix.Prepare (matrix.go:111-115). */
int cq_prepare(cq_matrix *m);
/* Matrix.Bytes (matrix.go:121-129): the reference's accounting. */
long long cq_bytes(const cq_matrix *m);
/* Device memory the matrix's storage holds (no reference counterpart). */
long long cq_device_bytes(const cq_matrix *m);
/* Matrix.Rows (matrix.go:133-145): a view of rows [lo, hi) sharing storage. */
int cq_rows(const cq_matrix *m, int lo, int hi, cq_matrix **view);
/* Matrix.Exact (matrix.go:152-157): a view whose products use the float
 * nibble tables (kernel.go:239-374) instead of the lut kernel. */
int cq_exact(const cq_matrix *m, cq_matrix **view);
/* A view sharing m's storage whose products of 16 or more activations run
 * Exact's semantics as a dense fp32 MFMA contraction: the activations
 * rotated as Exact rotates them (kernel.go:203-217), times W[r][k] =
 * norm[r][k/G] * codebook[index(r, k)] dequantized tile by tile into LDS, on
 * v_mfma_f32_32x32x2_f32. The sums run in the MFMA's order, so results are
 * within float32 rounding of Exact's (tests hold them within 1e-5 of the
 * largest |y| of each activation), not bit for bit; fewer activations,
 * and groups outside 32..1024, run Exact's nibble kernels. No counterpart in the
 * reference: for batched encoder-frame products that take Exact's
 * arithmetic at matrix-core rates. Rows views keep the setting; cq_exact
 * of it is a plain Exact view. */
int cq_dense(const cq_matrix *m, cq_matrix **view);
/* Name of the kernel the matrix's products run: "lut", "nibble4" or, for a
 * Dense view, "dense-f32" (kernel.go:30-43, 92-98). */
const char *cq_kernel_name(const cq_matrix *m);

/* Matrix.Row (matrix.go:161-181): row r dequantised as cact.CQ does, bit
 * for bit; dst holds In floats (host). */
int cq_row(const cq_matrix *m, float *dst, size_t dst_len, int r);
/* Matrix.GEMM (kernel.go:85-87); GEMV (kernel.go:78-80) is rows = 1.
 * x is [rows][In], dst [rows][Out], host row-major. */
int cq_gemm(const cq_matrix *m, float *dst, size_t dst_len, const float *x, size_t x_len, int rows);
/* cq.GEMMs (kernel.go:134-158): dsts[k] = ms[k].GEMM of the same x. */
int cq_gemms(int n, cq_matrix *const *ms, float *const *dsts, const size_t *dst_lens, const float *x, size_t x_len,
             int rows);

/* Device-pointer forms of GEMM, GEMMs and Row: every pointer is device
 * memory, work is queued on `stream` (a hipStream_t; NULL = the null
 * stream) and the call returns without waiting. */
int cq_gemm_dev(const cq_matrix *m, float *dst, const float *x, int rows, void *stream);
/* The same product, always in the MFMA form of the lut kernel (one-hot
 * indices times int8 table planes on v_mfma_i32_32x32x32_i8, exact int32
 * sums, the lut fold), bit for bit cq_gemm_dev's result. No counterpart in
 * the reference: the encoder's batched products (many frames at once) call
 * it; cq_gemm_dev picks it by itself when its grid is large enough. Group
 * 128, 2 or 4 bits, not an Exact view; else CQ_ERR_UNSUPPORTED. */
int cq_gemm_mfma_dev(const cq_matrix *m, float *dst, const float *x, int rows, void *stream);
/* The kernel cq_gemm_dev runs for `rows` activations: "lut", "lut-mfma",
 * "lut-mfma-tab" (the table pre-pass and its MFMA product), "lut-mfma-split",
 * "dense-f32" (a Dense view's fp32 MFMA form) or "nibble4". */
const char *cq_gemm_path(const cq_matrix *m, int rows);
int cq_gemms_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows, void *stream);
/* Bytes of device memory the workspace pool holds on every device (leased,
 * idle and held for graphs). No reference counterpart (the Go code's
 * scratch comes from a sync.Pool, internal/cq/kernel.go:59-74). */
long long cq_workspace_held(void);
/* Frees the idle workspaces whose work has completed, on every device;
 * returns the bytes still held. No reference counterpart. */
long long cq_workspace_trim(void);
/* cq_gemms_dev with the decode step's neighbours fused into the product
 * (no reference counterpart: one launch instead of three, results bit for
 * bit those of the separate steps). norm_gain non-null: every input row is
 * first ZCRMSNorm.Apply'd with that gain (internal/needle/norm.go:53-109).
 * resid non-null (n = 1): dst = resid + product, the residual add of the
 * decoder's layer body (resid may be dst). act 1 (no resid): dst =
 * silu(product), the synthetic decoder's FFN activation (as nd_silu_dev).
 * lut matrices only. */
int cq_gemms_fused_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows,
                       const float *norm_gain, const float *resid, int act, void *stream);
/* The gated attention's output projection: dst = product of (x * gate')
 * with gate' = sigmoid(gate) elementwise, sigmoid float32(1 / (1 +
 * exp(-float64(g)))) -- Attention.output (internal/needle/attention.go:
 * 242-260) and the cross-attention's gate (internal/decoder/cross.go:
 * 231-252) followed by outProj.Apply, one launch instead of two, bit for bit
 * nd_sigmoid_gate_dev then cq_gemms_dev. gate has x's layout (rows of the
 * matrices' input width) and is only read. resid non-null (n = 1): dst =
 * resid + product (resid may be dst). lut matrices only. */
int cq_gemms_gated_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, const float *gate, int rows,
                       const float *resid, void *stream);
/* cq_gemms_fused_dev (norm_gain only) whose outputs are also appended to
 * int8 row caches: the decoder's K and V projections followed by
 * Int8Rows.Append (internal/needle/int8.go:36-55; Attention.Extend's
 * projections, RoPE and append, internal/needle/cache.go:90-125), one launch instead of
 * three, results bit for bit kv_append_rope_dev's. No reference
 * counterpart. For k with kv_q[k] non-null, activation b's product row is
 * quantized per 64-wide head into row pos[b] of stream b's cache (codes
 * kv_q[k] + b*q_stride + pos[b]*out, scales kv_s[k] + b*s_stride +
 * pos[b]*out/64; no append where pos[b] is outside [0, cap)), after RoPE
 * at pos[b] with the half-width tables cos_t[k], sin_t[k] when cos_t and
 * cos_t[k] are non-null (internal/needle/rope.go:69-81). dsts[k] still
 * receives the product. Matrix k's view must cover whole 64-row blocks;
 * at most 8 lut matrices of one group size and index width (else
 * CQ_ERR_MISUSE / CQ_ERR_UNSUPPORTED). */
int cq_gemms_append_dev(int n, cq_matrix *const *ms, float *const *dsts, const float *x, int rows,
                        const float *norm_gain, int8_t *const *kv_q, float *const *kv_s, long long q_stride,
                        long long s_stride, const int32_t *pos, int cap, const float *const *cos_t,
                        const float *const *sin_t, void *stream);
/* A product chained to the next one through its tables (no reference
 * counterpart: the decoder's layer body, internal/decoder/decoder.go:
 * 446-505, runs each projection on the previous one's output; here the
 * previous product's launch also builds the next product's lookup tables,
 * lut.go:158-282, which that product would otherwise build in a launch of
 * its own). Results bit for bit those of the unchained calls.
 *
 * cq_tables_bytes: bytes of the tables of the product over next[0..n) at
 * `rows` activations, or 0 when that product takes no tables from a buffer
 * (it then runs as cq_gemms_fused_dev / cq_gemms_append_dev would). */
size_t cq_tables_bytes(int n, cq_matrix *const *next, int rows);
/* dst = [resid +] product of m and (x [* sigmoid(gate)]), as
 * cq_gemms_gated_dev (gate may be null: no gate); and, where the product
 * runs one workgroup per activation over all of m's rows, the tables of
 * the next product over next[0..n_next) of ZCRMSNorm(dst; next_gain)
 * (next_gain null: dst itself) into `tables`, tables_bytes =
 * cq_tables_bytes(n_next, next, rows) (0: none asked). *built = 1 when the
 * tables were built, else 0: then the next product runs unchained. The
 * next matrices take m's outputs as inputs. Calls that overlap on one
 * table buffer race. */
int cq_gemm_tables_dev(const cq_matrix *m, float *dst, const float *x, const float *gate, int rows, const float *resid,
                       int n_next, cq_matrix *const *next, const float *next_gain, void *tables, size_t tables_bytes,
                       int *built, void *stream);
/* The product over ms[0..n) of the activations whose tables
 * cq_gemm_tables_dev built (with `next` ms, or matrices of the same
 * codebook and geometry, and the same rows), with the epilogues of
 * cq_gemms_fused_dev (resid, act) and cq_gemms_append_dev (kv_q null: no
 * appends). The norm and the input are those the tables were built from.
 * CQ_ERR_MISUSE where cq_tables_bytes(n, ms, rows) is 0 or differs from
 * tables_bytes. */
int cq_gemms_tables_dev(int n, cq_matrix *const *ms, float *const *dsts, int rows, const float *resid, int act,
                        int8_t *const *kv_q, float *const *kv_s, long long q_stride, long long s_stride,
                        const int32_t *pos, int cap, const float *const *cos_t, const float *const *sin_t,
                        const void *tables, size_t tables_bytes, void *stream);
int cq_row_dev(const cq_matrix *m, float *dst, int r, void *stream);
/* Rows gathered by index: dst[i] = scale * Row(rows[i]) for i < n, rows a
 * device int32 array: the decoder's scaled token-embedding lookup for
 * several streams (internal/decoder/decoder.go:269-275) in one launch. A
 * listed row outside the matrix gives zeros. */
int cq_row_gather_dev(const cq_matrix *m, float *dst, const int32_t *rows, int n, float scale, void *stream);

/* Batch plans (no reference counterpart; the device-resident form of many
 * independent Matrix.GEMM calls): job k multiplies ms[k] by rows[k]
 * activations at device xs[k] into device ys[k], as cq_gemm_dev would, bit
 * for bit. cq_batch_new validates the jobs and uploads a device job table
 * once; cq_batch_run queues one lut-kernel launch per kernel geometry (index
 * width and group size) on `stream`, and can be captured in a HIP graph. The
 * matrices and buffers must outlive the plan's runs. Jobs on Exact views or
 * on groups the lut kernel does not hold in LDS return CQ_ERR_UNSUPPORTED. */
typedef struct cq_batch cq_batch;
int cq_batch_new(int n, cq_matrix *const *ms, float *const *ys, const float *const *xs, const int *rows,
                 cq_batch **plan);
int cq_batch_run(const cq_batch *plan, void *stream);
int cq_batch_launches(const cq_batch *plan);
void cq_batch_free(cq_batch *plan);

/* ---- int8 KV numerics (internal/needle/int8.go) ------------------------- */

/* QuantizeRows (int8.go:116-121, Append :125-141): x is rows of cols
 * floats; each chunk of width values gets its codes and one scale as
 * QuantizeRow (int8.go:36-55) gives them, bit for bit. Host and device
 * forms. */
int kv_quantize_rows(int8_t *q, float *s, const float *x, int rows, int cols, int width);
int kv_quantize_rows_dev(int8_t *q, float *s, const float *x, int rows, int cols, int width, void *stream);
/* KVCache.Fork for many streams at once (internal/needle/cache.go:62-67,
 * Int8Rows.Clip int8.go:155-161; the beams of internal/search/beam.go):
 * stream b of the int8 cache (codes q, scales s; streams of cap rows of
 * cols codes, width codes per scale) becomes the first len[b] rows of
 * stream parent[b], after which every stream extends on its own. parent
 * and len are device int32 arrays of `streams`; rows past len[b] are left
 * as they were. The reference shares the rows until one side appends
 * (copy on write); here they are copied, through the caller's temporaries
 * tmp_q, tmp_s of the cache's size. No reference counterpart as one call. */
int kv_reorder_dev(int8_t *q, float *s, int8_t *tmp_q, float *tmp_s, const int32_t *parent, const int32_t *len,
                   int streams, int cap, int cols, int width, void *stream);
/* kv_reorder_dev without the temporaries and without any allocation: the
 * temporaries live in a device array of 16 MiB that the library holds on
 * each GPU it runs on until the process ends. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, a serving loop's beam reorder, harnesses that
 * forbid hipMalloc). A reorder whose temporaries (streams * cap * cols
 * codes, 256-byte aligned, plus streams * cap * cols/width float scales)
 * exceed 16 MiB returns CQ_ERR_MISUSE. Every call on one GPU uses that
 * GPU's one array: calls that overlap on one GPU race. */
int kv_reorder_noalloc_dev(int8_t *q, float *s, const int32_t *parent, const int32_t *len, int streams, int cap,
                           int cols, int width, void *stream);

/* AttendInt8Spans (int8.go:208-272) on device memory for `batch`
 * independent streams (beam hypotheses, internal/search/beam.go:508-521).
 * Stream b reads q + b*q_stride (t rows of heads*qk floats), its keys and
 * values at kq + b*kv_stride codes (nk rows of k_cols / v_cols) with scales
 * at ks/vs + b*s_stride, its spans at spans + b*t*4 (per query row the
 * two ascending disjoint key spans {lo0, hi0, lo1, hi1}), and writes t rows
 * of heads*vd floats at out + b*out_stride (out_stride and q_stride 0 mean
 * dense streams; kv_stride and s_stride 0 share one cache). nk_max is the
 * number of key rows each stream's arrays hold: spans outside [0, nk_max)
 * leave that output untouched. quant_q chooses the int8 query
 * (int8Logits, int8.go:278-285) or the float32 query (dotsF32I8,
 * int8.go:289-300). The softmax is softmaxInPlace (load.go:128-138) with
 * the amd64 kernel's exponent (exp_amd64.s:68-124). */
int kv_attend_int8_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                       const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                       int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans, int nk_max,
                       float scale, int quant_q, int batch, void *stream);
/* The same with the query heads first rotated by RoPE (Rope.apply,
 * internal/needle/rope.go:69-81) at row qpos[b*t + i] of the (positions x
 * qk/2) cos/sin tables: Attention.Extend's rotated query
 * (internal/needle/attention.go:345-415) without a separate pass. */
int kv_attend_int8_rope_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                            const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                            int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans,
                            int nk_max, float scale, int quant_q, int batch, const float *cos_t, const float *sin_t,
                            const int32_t *qpos, void *stream);
/* kv_attend_int8_dev over caches that streams share: stream b reads the
 * keys and values of cache kv_index[b] (a device int32 array of `batch`),
 * one of kv_streams caches kv_stride codes / s_stride scales apart; an
 * index outside [0, kv_streams) leaves stream b's output untouched. The
 * beams of one utterance after State.Fork (internal/decoder/decoder.go:
 * 223-240) share its cross-attention memory, which is never copied. */
int kv_attend_int8_shared_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                              const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                              int v_cols, int vd, long long kv_stride, long long s_stride, const int32_t *spans,
                              int nk_max, float scale, int quant_q, int batch, const int32_t *kv_index, int kv_streams,
                              void *stream);

/* Int8Rows.Append (int8.go:125-141) on a device KV cache for `batch`
 * streams: stream b's row x + b*cols is quantised per chunk of width
 * (QuantizeRow, bit for bit) into codes q + b*q_stride + pos[b]*cols and
 * scales s + b*s_stride + pos[b]*(cols/width); pos is a device array, and a
 * position outside [0, cap) is skipped. */
int kv_append_dev(int8_t *q, float *s, const float *x, int batch, int cols, int width, long long q_stride,
                  long long s_stride, const int32_t *pos, int cap, void *stream);
/* The same with each chunk (a key head) first rotated by RoPE (rope.go:
 * 69-81) at row pos[b] of the (positions x width/2) cos/sin tables: the
 * rotated key appended (attention.go:345-415). width <= 256, even. */
int kv_append_rope_dev(int8_t *q, float *s, const float *x, int batch, int cols, int width, long long q_stride,
                       long long s_stride, const int32_t *pos, int cap, const float *cos_t, const float *sin_t,
                       void *stream);

/* ---- float blocks of a decode step, on device memory -------------------- */

/* ZCRMSNorm.Apply (internal/needle/norm.go:53-66, meanSquare :91-109):
 * dst = gain * x / sqrt(mean(x^2) + 1e-6) per row of dim, mean in float64
 * as the reference sums it; gain = 1 + scale (NewZCRMSNorm, norm.go:22-30).
 * dst may be x. */
int nd_zcrmsnorm_dev(float *dst, const float *x, const float *gain, int rows, int dim, void *stream);
/* Rope.apply (internal/needle/rope.go:69-81) in place on rows of heads
 * vectors of head_dim: row r uses position pos[r / rows_per_pos] of the
 * (positions x head_dim/2) cos/sin tables (NewRope, rope.go:17-44). A row
 * whose position is outside [0, positions) is left unchanged (the
 * reference's table slice would panic there). */
int nd_rope_dev(float *x, int rows, int heads, int head_dim, const float *cos_t, const float *sin_t, int positions,
                const int32_t *pos, int rows_per_pos, void *stream);
/* argmax (internal/decoder/greedy.go:181-191) of each row of n: the first
 * index of the largest value. */
int nd_argmax_dev(int32_t *out, const float *v, int rows, int n, void *stream);
/* nd_argmax_dev that also advances each stream's decode position, the end
 * of Decoder.Extend's step (internal/decoder/decoder.go:252-302, greedy.go:
 * 31-69): pos[r] += 1, and span_hi[r * span_stride] = pos[r] + 1, the key
 * bound of the next step's self-attention after its append. No reference
 * counterpart as one call: the device decode step's bookkeeping without
 * launches of its own. */
int nd_argmax_advance_dev(int32_t *out, const float *v, int rows, int n, int32_t *pos, int32_t *span_hi,
                          int span_stride, void *stream);
/* nd_argmax_advance_dev with greedy decoding's stop (internal/decoder/
 * greedy.go:50-66): a stream whose done[r] is nonzero is left as it is (its
 * token, position and key bound); otherwise, after the argmax and the
 * advance, done[r] = 1 when the token is eos. Streams of one batch stop one
 * by one, each after its own EOS, as GreedyMemory stops each hypothesis. */
int nd_argmax_advance_eos_dev(int32_t *out, const float *v, int rows, int n, int32_t *pos, int32_t *span_hi,
                              int span_stride, int32_t *done, int eos, void *stream);
/* x = x * sigmoid(x), sigmoid from the amd64 exponent kernel's arithmetic
 * (exp_amd64.s:84-112) on non-positive arguments. No reference
 * counterpart: the synthetic decoder's FFN activation. */
int nd_silu_dev(float *x, long long n, void *stream);
/* fakeQuant (internal/needle/int8.go:57-75): rows of cols values, each
 * chunk of width through QuantizeRow and back, dst = float32(q) * s; the
 * input of a Linear WithInt8Input (quantInput, int8.go:81-88;
 * internal/needle/linear.go:82-86). dst may be x. */
int nd_fake_quant_dev(float *dst, const float *x, long long rows, int cols, int width, void *stream);
/* x += y elementwise (the residual adds). */
int nd_add_dev(float *x, const float *y, long long n, void *stream);
/* HadamardMLP.Forward (internal/needle/hadamard.go:172-294), Whistle's
 * Monarch FFN, on rows of dim values: cond = 1 + softmax(x cond_v) cond_u;
 * z1 = kron(d1 x; w1a, w1b)[p1]; z2 = kron(silu(d2 cond z1 + b2); w2a,
 * w2b)[p2]; out = d4 kron(d3 z2; w3a, w3b), kron(z; a, b) = a^T Z b with Z
 * the na x nb matrix of z (kronApply, hadamard.go:296-310); x zero-padded
 * to n = na * nb >= dim, out cut back to dim (LoadHadamardMLP's padding,
 * hadamard.go:19-24). vecs = {d1, d2, b2, d3, d4} (n each), factors =
 * {w1a, w1b, w2a, w2b, w3a, w3b} row-major, cond_v dim x rank, cond_u
 * rank x n, p1 and p2 permutations of n (hada_p1/p2). n <= 1024, rank <= 32.
 * Float32, within 1e-5 of the float64 form (hadamard_test.go:152-191); the
 * reference's GEMMs sum in their library's own order. */
int nd_hadamard_mlp_dev(float *out, const float *x, int rows, int dim, int na, int nb, int rank,
                        const float *const *vecs, const float *const *factors, const float *cond_v,
                        const float *cond_u, const int32_t *p1, const int32_t *p2, void *stream);
/* RMSUnit (internal/needle/norm.go:68-81): each row of dim times
 * float32(1 / sqrt(float64(meanSquare + 1e-6))), meanSquare in float64 as
 * ZCRMSNorm's; mHC's nx of the lane stream (rows of lanes * dim). */
int nd_rms_unit_dev(float *dst, const float *x, int rows, int dim, void *stream);
/* MHC.forward's heads and block input (internal/needle/mhc.go:204-219,
 * 246-263) from the φ products' logits (rows x lanes, rows x lanes x
 * lanes): with affine non-null (device floats {a_pre, a_post, a_res,
 * b_pre[lanes], pre_off[lanes], b_post[lanes], post_off[lanes],
 * b_res[lanes^2]}) the logits are first a * logit + b (+ off) as MHC.logits
 * rounds them; h_pre = sigmoid, h_post = 2 sigmoid, h_res = sinkhorn of 20
 * iterations (mhc.go:301-417), u[i] = sum_k h_pre[k] stream[i, k] in k
 * order (stream rows x lanes x dim, u rows x dim). lanes <= 8. */
int nd_mhc_heads_dev(float *h_pre, float *h_post, float *h_res, float *u, const float *pre_logits,
                     const float *post_logits, const float *res_logits, const float *stream_rows, int rows, int lanes,
                     int dim, const float *affine, void *stream);
/* nd_mhc_heads_dev with the three φ products' logits in one array, rows x
 * (2 lanes + lanes^2): pre, post, then res of each row, as one product of
 * the three φ matrices stacked row-wise gives them (the same outputs bit
 * for bit; one table build per activation instead of three). */
int nd_mhc_heads_stacked_dev(float *h_pre, float *h_post, float *h_res, float *u, const float *logits,
                             const float *stream_rows, int rows, int lanes, int dim, const float *affine,
                             void *stream);
/* MHC.forward's output (internal/needle/mhc.go:229-234, 266-299): y =
 * block_out - u, out[i, a] = sum_b h_res[i, a, b] stream[i, b] (b in order)
 * + h_post[i, a] y. out must not be the stream. */
int nd_mhc_mix_dev(float *out, const float *stream_rows, const float *h_res, const float *h_post,
                   const float *block_out, const float *u, int rows, int lanes, int dim, void *stream);
/* AttendInt8Spans over paged int8 caches: the arrays kq/ks/vq/vs are one
 * pool of pool_pages pages of page_rows rows (a power of two; codes k_cols /
 * v_cols per row, scales per head), and key j of stream b is row
 * pages[b*page_stride + j/page_rows]*page_rows + j%page_rows. Otherwise
 * kv_attend_int8_rope_dev (cos_t null: no RoPE of the query). Forked
 * streams share their full pages without a copy, as KVCache.Fork shares the
 * rows so far until one side appends (internal/needle/cache.go:62-67). An
 * entry outside [0, pool_pages) reads page 0. */
int kv_attend_int8_paged_dev(float *out, long long out_stride, const float *q, long long q_stride, int t, int heads,
                             const int8_t *kq, const float *ks, int k_cols, int qk, const int8_t *vq, const float *vs,
                             int v_cols, int vd, const int32_t *spans, int nk_max, float scale, int quant_q, int batch,
                             const float *cos_t, const float *sin_t, const int32_t *qpos, const int32_t *pages,
                             int page_stride, int page_rows, int pool_pages, void *stream);
/* Attention.Extend's steps between the projections and the attention for
 * one token per stream (internal/needle/cache.go:88-125): q, k, v are batch
 * rows of dim (heads of 64) at positions pos[b]. In order: the causal taps
 * (taps > 0; applyTaps on extendTaps' rows, attention.go:597-613,
 * cache.go:143-154): out = sum_j taps_w[z][j] * row(pos - j) over j <= pos,
 * from 0 in j order, products rounded; hist [batch][taps][3][dim] holds the
 * raw rows of the last positions at slot position mod taps and is updated
 * (slot pos[b] mod taps, which the step does not read: running a position
 * again gives the same result); the per-head ZCRMSNorm of q and k (q_gain / k_gain of 64; null:
 * none; normRotate, attention.go:298-330); RoPE of k at pos[b] (cos_t null:
 * none; tables of 32 per row, `positions` rows); then k and v quantized per
 * head and appended at row pos[b] (< cap) through the page table (as
 * kv_attend_int8_paged_dev reads them; an entry outside the pool skips the
 * append). q is written back, normed and not rotated (the attention rotates
 * it). dim a multiple of 64 up to 1024. No reference counterpart as one call. */
int nd_qkv_prep_dev(float *q, const float *k, const float *v, int batch, int dim, float *hist, const float *taps_w,
                    int taps, const float *q_gain, const float *k_gain, const float *cos_t, const float *sin_t,
                    int positions, const int32_t *pos, int cap, int8_t *kq, float *ks, int8_t *vq, float *vs,
                    const int32_t *pages, int page_stride, int page_rows, int pool_pages, void *stream);
/* h = resid + float32(scale * ZCRMSNorm(y)) per row of dim (resid null or
 * h: h += ...): the attention's post norm and residual factor, h +=
 * float32(gate * postNorm(a)) (internal/needle/block.go:183-188), and the
 * cross branch's (internal/decoder/cross.go:255-263 with the hook's add,
 * decoder.go:461-465). y is only read. dim a multiple of 256 up to 4096. */
int nd_norm_scaled_add_dev(float *h, const float *resid, const float *y, const float *gain, float scale, int rows,
                           int dim, void *stream);
/* RMSUnit (internal/needle/norm.go:68-81) of each row of dim, then its
 * fakeQuant as one chunk (int8.go:57-75): the mHC phi products' int8 input
 * (mhc.go:99-106 with Linear.WithInt8Input, linear.go:80-87), one launch,
 * bit for bit nd_rms_unit_dev then nd_fake_quant_dev. dim a multiple of 256
 * up to 4096; dst may be x. */
int nd_rms_unit_quant_dev(float *dst, const float *x, int rows, int dim, void *stream);
/* ExpandLanes / CollapseLanes (internal/needle/mhc.go:137-170): each row of
 * x to `lanes` equal lanes of the stream (rows x lanes x dim), and back as
 * the lane mean (lanes summed in order from 0, then divided by lanes). */
int nd_expand_lanes_dev(float *stream_rows, const float *x, int rows, int lanes, int dim, void *stream);
int nd_collapse_lanes_dev(float *x, const float *stream_rows, int rows, int lanes, int dim, void *stream);
/* Page dst[j] of a paged int8 cache (page_rows rows of cols codes, cols/width
 * scales) becomes a copy of page src[j], j < n: the copy-on-write of a
 * forked stream's partly filled page. Pairs outside [0, pool_pages) are
 * skipped. No reference counterpart (its Fork copies on the next append). */
int kv_page_copy_dev(int8_t *q, float *s, const int32_t *src, const int32_t *dst, int n, int page_rows, int cols,
                     int width, int pool_pages, void *stream);
/* dst row r = src row idx[r] (idx null: r), rows of width floats: a fork's
 * tap history (State.Fork shares it, decoder.go:218-240). dst must not
 * overlap src. */
int nd_gather_rows_dev(float *dst, const float *src, const int32_t *idx, int rows, long long width, void *stream);
/* The attention's output gate (internal/needle/attention.go:245-249):
 * gate[i] = sigmoid(gate[i]), out[i] *= gate[i], sigmoid being jax.nn.sigmoid
 * in float32 as the reference writes it, float32(1 / (1 + exp(-float64(x))))
 * (internal/needle/load.go:120-123; internal/decoder/cross.go:240-248). */
int nd_sigmoid_gate_dev(float *out, float *gate, long long n, void *stream);

#ifdef __cplusplus
}
#endif

#endif
