/* CPU oracle for the qpack Llama token loop: a plain-C restatement of the reference's x86 CPU path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker.  The product path (qpack_amd/) never links, loads or calls it.
 *
 * Every function names the reference lines it restates.  Floating-point operations follow the reference's evaluation
 * order as compiled by g++ -O3 -mavx2 -mfma (the reference's own portable build): 8-lane AVX2 accumulators are emulated
 * lane by lane, and every multiply-add that g++ contracts into an FMA is an explicit fmaf() here (the oracle itself is
 * compiled with -ffp-contract=off).
 */
#ifndef QPACK_ORACLE_H
#define QPACK_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_Q8 = 0, OR_Q4 = 1, OR_F32 = 2, OR_Q1 = 3 };
#define OR_QB 128          /* activation block, /root/reference/src/kernels_impl.h:13 */
#define OR_ACT_MAX 32767.f /* kActMax on x86, /root/reference/src/kernels_impl.h:19 */

/* a weight matrix: q8 = int8 [rows, cols] + f32 scale [rows]; q4 = u8 [rows, cols/2] + f16 scale [rows, cols/32];
 * q1 = sign bits u8 [rows, G * 16] + f16 scale [rows, G], G = ceil(cols / 128); f32 = float [rows, cols] (s unused) */
typedef struct { int kind, rows, cols; const void *q; const void *s; } or_mat;

typedef struct {
  int d, L, nh, nkv, hd, ff, V, ctx, tied;
  float eps;
  double theta;
} or_cfg;

typedef struct {
  const float *attn_norm, *ffn_norm, *bq, *bk, *bv; /* biases may be NULL */
  or_mat wq, wk, wv, wo, wg, wu, wd;
} or_layer;

typedef struct or_model or_model;

/* fp16 <-> fp32, round to nearest even (F16C semantics used by /root/reference/src/kernels_x86.cpp:449-452) */
uint16_t or_f32_to_f16(float f);
float or_f16_to_f32(uint16_t h);

/* activation quantisation of one vector: quant_rows, /root/reference/src/kernels.cpp:17-31 */
void or_quant_act(const float *x, int cols, int16_t *xq, float *bs);
/* exact int32 dot products per (row, 128-column block) for q8 and per (row, 32-column group) for q4: the integer
 * accumulators inside rows_q8 / rows_q4 (/root/reference/src/kernels_x86.cpp:57-63, :85-101) */
void or_block_sums_q8(const int8_t *Q, int rows, int cols, const int16_t *xq, int32_t *out);
void or_group_sums_q4(const uint8_t *Q, int rows, int cols, const int16_t *xq, int32_t *out);
/* the row kernels on quantised activations: rows_q8 / rows_q4, /root/reference/src/kernels_x86.cpp:55-106 */
void or_rows_q8(const int8_t *Q, const float *scale, const int16_t *xq, const float *bs, float *y, int rows, int cols);
void or_rows_q4(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int rows, int cols);
/* q1 (sign bits, groups of 128 columns): rows_q1, /root/reference/src/kernels_x86.cpp:167-203; the exact int32 dot
 * product of every (row, group) with the int16 activation (columns past cols read as 0) */
void or_rows_q1(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int rows, int cols);
void or_group_sums_q1(const uint8_t *Q, int rows, int cols, const int16_t *xq, int32_t *out);
/* matvec (kernels.cpp:72-96) and the tiled prompt product matmul (kernels.cpp:124-143 -> mm_q8 / mm_q4,
 * kernels_x86.cpp:287-371); Y is [B, rows] */
void or_matvec(const or_mat *W, const float *x, float *y);
void or_matmul(const or_mat *W, const float *X, int B, float *Y);
/* elementwise helpers */
void or_rmsnorm(const float *x, const float *w, int n, float eps, float *out); /* kernels.cpp:184-189 */
void or_exp_v(const float *x, float *y, int n);                                 /* kernels_x86.cpp:406-421 */
void or_silu_mul(float *g, const float *u, int n);                              /* kernels_x86.cpp:427-434 */
void or_row_f32(const or_mat *W, int r, float *out);                            /* kernels.cpp:146-162 */

/* the Llama model: /root/reference/src/model_llama.cpp:20-201 */
or_model *or_create(const or_cfg *cfg, const or_mat *embed, const or_mat *head, const float *final_norm,
                    const or_layer *layers);
void or_free(or_model *m);
void or_reset(or_model *m);
int or_pos(const or_model *m);
int or_set_pos(or_model *m, int pos);
/* want: 0 state only, 1 logits [V] into out, 2 final normed hidden [d] into out.  Return 0, or -1 on a bad token /
 * full context (the reference throws there, model_llama.cpp:169-170) */
int or_step(or_model *m, int tok, int want, float *out);
int or_prefill(or_model *m, const int *toks, int n, int want, float *out);
int or_greedy(or_model *m, int tok, int n, int *out);
/* the fp16 KV cache [L][ctx][nkv*hd] for K and V */
uint16_t *or_kcache(or_model *m);
uint16_t *or_vcache(or_model *m);
void or_set_threads(int n);
/* the sampler's top-M candidates (top_m + sort, /root/reference/src/sampler.cpp:12-27, :41-42) */
int or_top_m(const float *x, int V, int M, int *idx, float *val);
/* evaluation-order variants for experiments (0 = the reference's orders everywhere) */
enum { OR_ORD_TREE_NORM = 1, OR_ORD_ROWS_PREFILL = 2, OR_ORD_ATTN_F64 = 4, OR_ORD_EXP_F64 = 8 };
void or_set_order(int flags);

/* QPACK3 static rANS codec (/root/reference/include/qpack/rans.h; format in /root/reference/QPACK2.md:30-51).
 * Errors: OR_RANS_* (negative); the reference throws std::runtime_error at the same points. */
enum { OR_RANS_TRUNCATED = -1, OR_RANS_BAD_TABLE = -2, OR_RANS_OVERRUN = -3, OR_RANS_BAD_CODEC = -4, OR_RANS_CAPACITY = -5,
       OR_RANS_NORMALISE = -6, OR_RANS_TRUNCATED_PLANE = -7, OR_RANS_SHORT = -8, OR_RANS_SHORT_CHUNKED = -9,
       OR_RANS_TRUNCATED_TABLE = -10, OR_RANS_TRUNCATED_CHUNK = -11 };
/* raw (decoded) length of a blob, or an error (rans.h:75) */
int64_t or_rans_raw_size(const uint8_t *p, int64_t len);
/* a plain (codec 1 / 2) or chunked (codec 3) blob -> its raw bytes; out must hold or_rans_raw_size bytes (rans.h:101-113) */
int or_rans_decode(const uint8_t *p, int64_t len, uint8_t *out, int64_t cap);
/* raw bytes -> a plain codec 1 (planes 1..4) or codec 2 blob; returns the blob length or an error (rans.h:21-49, :81-93) */
int64_t or_rans_encode(const uint8_t *raw, int64_t n, int codec, int planes, uint8_t *out, int64_t cap);
/* the encoder's 12-bit frequency table for one plane of symbols (rans.h:23-37) */
int or_rans_freqs(const uint8_t *sym, int64_t n, int nsym, uint32_t *f);

#ifdef __cplusplus
}
#endif
#endif
