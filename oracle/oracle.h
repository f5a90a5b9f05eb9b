/*
 * CPU oracle for go-whistle's CQ quantized-matrix path and its int8 KV
 * numerics: a plain-C restatement of the reference's Go arithmetic, used as
 * the checker for the HIP library.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load liboracle.so. The product library
 * (libcqhip.so) neither links nor calls it.
 *
 * Every function names the reference file:line it follows. Build flags
 * (Makefile): -O2 -ffp-contract=off -fno-fast-math, so that every float32
 * multiply and add rounds on its own as in Go on amd64 (which never fuses).
 *
 * Pinning (what checks each function independently of this file) is listed
 * in the header comment of each source file; tests/test_oracle_*.py hold
 * the checks.
 */
#ifndef CQ_ORACLE_H
#define CQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Go's conversion of a float64 to int32 on amd64 (CVTTSD2SL): truncation,
 * and the integer indefinite 0x80000000 for a NaN or a value out of range
 * (C leaves that case undefined). int8(r) is its low byte: 0 for a NaN,
 * as arm64's FCVTZS gives too. */
static inline int32_t go_int32_of(double r) {
    if (r != r || r >= 2147483648.0 || r < -2147483648.0) return INT32_MIN;
    return (int32_t)r;
}
static inline int8_t go_int8_of(double r) { return (int8_t)(uint8_t)((uint32_t)go_int32_of(r) & 0xFFu); }

/* ---- internal/cact: the packed CQ form ---------------------------------- */

/* cact.Packed (internal/cact/packed.go:18-29): Out rows of RowBytes index
 * bytes (LSB-first bitstream of the group-padded row), Out*Groups FP16 norms
 * (little-endian, [out][groups]) and the 2^bits codebook. */
typedef struct {
    int out, in, group, bits, width; /* width: bits per stored index (Packed.Width) */
    const float *codebook;  /* 1 << bits levels */
    const uint8_t *index;   /* out * row_bytes */
    const uint8_t *norms;   /* 2 * out * groups */
    size_t index_len, norms_len, codebook_len;
} orc_packed;

float orc_f16_to_f32(uint16_t h);                      /* half.go:8-40 */
void orc_f16_to_f32_n(float *dst, const uint16_t *h, size_t n);
void orc_unpack_lsb(uint8_t *idx, const uint8_t *packed, int n, int width); /* cq.go:124-137 */
void orc_fwht(float *x, int n);                        /* cq/kernel.go:384-393 */
/* cact.CQ: the dequantised [out][in] matrix (internal/cact/cq.go:67-118). */
int orc_cq_dequant(float *w, const orc_packed *p);

/* ---- internal/cq: Matrix ------------------------------------------------ */

typedef struct orc_matrix orc_matrix;

/* cq.New / cq.NewGather (internal/cq/matrix.go:46-96). Returns NULL and
 * writes a "cq: ..." message to err (if non-NULL, errlen bytes) on bad
 * input. The matrix copies everything it needs. */
orc_matrix *orc_new(const orc_packed *p, char *err, size_t errlen);
void orc_free(orc_matrix *m);
/* Matrix.Rows (matrix.go:131-145): a view sharing storage; NULL on a bad
 * range. Views must be freed with orc_free and before their root. */
orc_matrix *orc_rows(const orc_matrix *m, int lo, int hi);
int orc_out(const orc_matrix *m);
int orc_in(const orc_matrix *m);

enum { ORC_GATHER = 0, ORC_NIBBLE = 1, ORC_NIBBLE4 = 2, ORC_LUT = 3 };

/* Matrix.gemm with the named kernel (kernel.go:100-125): dst [rows][out],
 * x [rows][in]. Returns -1 on a shape mismatch (the reference panics). */
int orc_gemm(const orc_matrix *m, int kernel, float *dst, const float *x, int rows);
/* cq.GEMMs (kernel.go:134-158): all matrices must share the lut tables for
 * the shared path; otherwise each runs its own GEMM. kernel is ORC_LUT for
 * Matrix.GEMM's default on amd64 with AVX2, ORC_NIBBLE4 for Exact views. */
int orc_gemms(orc_matrix *const *ms, int n, int kernel, float *const *dsts, const float *x, int rows);
/* Matrix.Row (matrix.go:159-181). */
int orc_row(const orc_matrix *m, float *dst, int r);

/* The lut kernel's routines (internal/cq/lut.go), for direct tests. */
float orc_lut_tables2(uint8_t *tab, const float *x, int n, const float *cb, float cb_max); /* lut.go:239-258 */
float orc_lut_tables4(uint8_t *tab, const float *x, int n, const float *cb, float cb_max); /* lut.go:263-282 */
void orc_lut_lookup(float *y, const uint8_t *idx, const uint8_t *tab, const float *norm, const float *steps,
                    int blocks, int groups, int gb);                                       /* lut.go:289-313 */
float orc_lut_step(int group);                                                             /* lut.go:213-215 */

/* The AVX2 forms of the lut routines (lut_amd64.s, cq_avx2.c), bit for bit
 * the generic ones; callable only where orc_have_avx2(). fwht: n a power of
 * two >= 8; tables: n a multiple of 8. */
int orc_have_avx2(void);
void orc_fwht_avx2(float *x, int n);                                                        /* lut_amd64.s:12-75 */
float orc_lut_tables2_avx2(uint8_t *tab, const float *x, int n, const float *cb, float cb_max); /* :150-197 */
float orc_lut_tables4_avx2(uint8_t *tab, const float *x, int n, const float *cb, float cb_max); /* :199-233 */
void orc_lut_lookup_avx2(float *y, const uint8_t *idx, const uint8_t *tab, const float *norm, const float *steps,
                         int blocks, int groups, int gb);                                   /* :235-378 */
/* How lut products and the int8 attention run from here on: avx2 1 for the
 * AVX2 forms (-1 if the CPU lacks AVX2 or FMA), threads > 1 to split the lut
 * products as gemmLUT does (lut.go:102-201). Process-wide; not to be changed
 * while products run. */
int orc_set_cpu(int avx2, int threads);
int orc_cpu_avx2(void); /* the mode's avx2 flag */
/* The worker pool behind the split (cpu_pool.c): reserve keeps threads - 1
 * workers (-1 if one cannot start); run calls fn(ctx, lo, hi) on pieces
 * [n*p/pieces, n*(p+1)/pieces) of [0, n), piece 0 on the caller, and returns
 * when all are done. One caller thread at a time. */
typedef void (*orc_piece_fn)(void *ctx, int lo, int hi);
int orc_pool_reserve(int threads);
void orc_pool_run(int n, int pieces, orc_piece_fn fn, void *ctx);
/* The AVX2 forms of the int8 attention kernels (int8kernel_amd64.s,
 * exp_amd64.s; int8_avx2.c), bit for bit the generic ones; widths positive
 * multiples of 16, n8 a multiple of 8. AttendInt8Spans runs them in the
 * AVX2 mode. */
void orc_dots_i8_avx2(int32_t *dst, int n, const int8_t *q, int width, const int8_t *k, int stride);
void orc_axpys_i8_avx2(float *out, int width, const float *w, int n, const int8_t *v, int stride);
float orc_exp_sub_sum_avx2(float *s, int n8, float m);

/* ---- internal/needle: int8 numerics ------------------------------------- */

float orc_quantize_row(int8_t *q, const float *x, int n);                /* int8.go:36-55 */
void orc_quantize_rows(int8_t *q, float *s, const float *x, int rows, int cols, int width); /* int8.go:116-141 */
void orc_fake_quant(float *dst, const float *x, long rows, int cols, int width);          /* int8.go:62-75 */
void orc_dots_i8(int32_t *dst, int n, const int8_t *q, int width, const int8_t *k, int stride);   /* int8kernel.go:346-357 */
void orc_axpys_i8(float *out, int width, const float *w, int n, const int8_t *v, int stride);     /* int8kernel.go:360-368 */
void orc_dots_f32_i8(float *dst, int n, const float *q, int width, const int8_t *k, int stride); /* int8.go:289-300 */

/* expSubSum: variant 0 = expSubSumGeneric (exp.go:21-31), float64 exp per
 * value; variant 1 = the amd64 AVX2+FMA kernel's arithmetic on the
 * multiple-of-8 prefix plus the generic tail (exp_amd64.go:13-25,
 * exp_amd64.s:68-124). */
float orc_exp_sub_sum(float *s, int n, float m, int variant);
void orc_softmax(float *s, int n, int variant);                           /* load.go:125-138 */

/* AttendInt8Spans (int8.go:208-272). q: t rows of heads*qk floats; k codes
 * [nk][k_cols], k scales [nk][k_cols/qk]; v likewise with vd. spans: per
 * query row i, two ascending disjoint spans {lo0, hi0, lo1, hi1}. out: t rows
 * of heads*vd. probs (optional): [(i*heads+h)*nk + j]. */
int orc_attend_int8_spans(float *out, const float *q, int t, int heads, const int8_t *kq, const float *ks,
                          int k_cols, int qk, const int8_t *vq, const float *vs, int v_cols, int vd, int nk,
                          const int32_t *spans, float scale, int quant_q, int exp_variant, float *probs);

/* One lane of the amd64 exponent kernel (exp_amd64.s:84-112). */
float orc_exp_lane(float x);

/* ---- decode-step float blocks (step_oracle.c) --------------------------- */

void orc_zc_rmsnorm(float *dst, const float *x, const float *gain, int rows, int dim); /* norm.go:53-66 */
void orc_rope(float *x, int rows, int heads, int head_dim, const float *cos_t, const float *sin_t,
              const int32_t *pos);                                                    /* rope.go:69-81 */
void orc_argmax(int32_t *out, const float *v, int rows, int n);                          /* greedy.go:181-191 */
void orc_silu(float *x, long n);
double orc_exp64(double x);                             /* fdlibm e_exp.c; Go's portable math.Exp */
float orc_gate_sigmoid(float x);                        /* load.go:120-123, cross.go:322-325 */
void orc_sigmoid_gate(float *out, float *gate, long n); /* attention.go:245-249 */
void orc_rms_unit(float *dst, const float *x, int rows, int dim);                  /* norm.go:68-81 */
void orc_sinkhorn(float *k, int n, int iters);                                      /* mhc.go:301-417 */
void orc_mhc_heads(float *h_pre, float *h_post, float *h_res, float *u, const float *pre_l, const float *post_l,
                   const float *res_l, const float *stream, int rows, int n, int dim, const float *affine);
void orc_mhc_mix(float *out, const float *stream, const float *h_res, const float *h_post, const float *block_out,
                 const float *u, int rows, int n, int dim);                          /* mhc.go:229-299 */

/* ---- the synthetic decoder's greedy decode (decode_oracle.c) ------------ */

/* The matrices of a layer, in order: wq wk wv wg wo wcq wcg wco wck wcv w1
 * w2, then (with lanes) phi_pre phi_post phi_res. */
enum { ORC_DEC_NMATS = 15 };

typedef struct {
    int vocab, dim, heads, head_dim, ffn, layers, frames, max_pos;
    int taps;       /* causal taps on q/k/v (0: none) */
    int qk_norm;    /* per-head q/k ZCRMSNorm before RoPE */
    int post_norm;  /* the attention's post norm and residual factor */
    int cross_norm; /* the cross q norm, post norm and residual factor */
    int lanes;      /* mHC lanes around every layer (0: none) */
    float scale;    /* the embedding row's factor */
    orc_matrix *emb;                 /* vocab x dim, tied head */
    orc_matrix *const *mats;         /* layers x ORC_DEC_NMATS (unused slots NULL) */
    const float *gains;              /* (3 layers + 1) x dim: attention, cross, FFN norms; final */
    const float *rope_cos, *rope_sin; /* max_pos x head_dim/2 */
    const float *qk_gains;           /* layers x 4 x head_dim: self q, self k, cross q, cross k */
    const float *post_gains;         /* layers x 2 x dim: self, cross */
    const float *res_scale;          /* layers x 2: self, cross */
    const float *taps_w;             /* layers x 3 (q, k, v) x taps x dim */
    const float *mhc_affine;         /* layers x (3 + 4 lanes + lanes^2), orc_mhc_heads' affine */
} orc_dec_model;

/* One stream's int8 cross memory: per layer, frames key-major rows of dim
 * codes and heads scales (cross.project with Int8.KV, cross.go:181-204). */
typedef struct {
    const int8_t *const *kq;
    const float *const *ks;
    const int8_t *const *vq;
    const float *const *vs;
} orc_dec_memory;

typedef struct orc_dec_state orc_dec_state;
orc_dec_state *orc_dec_new(const orc_dec_model *m, const orc_dec_memory *mem); /* NewState (decoder.go:212-215) */
orc_dec_state *orc_dec_fork(const orc_dec_state *s);                           /* State.Fork (decoder.go:218-240) */
void orc_dec_free(orc_dec_state *s);
int orc_dec_len(const orc_dec_state *s);
/* Decoder.Extend of one token (decoder.go:248-302, 446-523): the next
 * token's logits (vocab floats, NULL: not kept); returns their argmax, or
 * -1 past max_pos or for a token out of range. */
int orc_dec_step(orc_dec_state *s, int token, float *logits);
/* GreedyMemory's loop (greedy.go:30-69) from `first`: up to n tokens, each
 * step's logits to logits[i] (NULL: not kept), stopping at eos (>= 0; not
 * written, *stopped = 1). Returns the count, -1 on a failed step. */
int orc_dec_greedy(orc_dec_state *s, int first, int n, int eos, int32_t *tokens, float *logits, int *stopped);
/* streams greedy decodes from fresh states, n tokens each (no stop), on
 * `threads` threads, a stream per thread at a time: tokens [streams][n],
 * counts [streams]. The lut products must run on one thread
 * (orc_set_cpu(.., 1)). */
int orc_dec_streams(const orc_dec_model *m, const orc_dec_memory *mems, int streams, const int32_t *first, int n,
                    int threads, int32_t *tokens, int32_t *counts);

#ifdef __cplusplus
}
#endif

#endif
