/* qpack_hip.h - C ABI of the MI355X (gfx950) Llama-family token loop.
 *
 * This is the drop-in boundary for qpack's GPU model (`LlamaCuda`, /root/reference/src/model_llama_cuda.cu:445-632),
 * selected by QPACK_DEVICE in load_model (/root/reference/src/model_llama.cpp:221-235).  Each model entry point replaces
 * one method of the C++ interface qp::Model (/root/reference/include/qpack/qpack.h:128-171); the reference-side adapter
 * a maintainer adds is a qp::Model subclass forwarding each method to these functions.
 *
 * Conventions
 *   - Every function returns int status: 0 = ok, -1 = error; qph_last_error() gives the calling thread's message.  The C++
 *     adapter turns a non-zero status into std::runtime_error, the reference's error convention.
 *   - Plain pointers and sizes only.  Host pointers unless a parameter says "device".
 *   - A model is not re-entrant: one host thread per model at a time (the reference's contract; qpack-server serialises
 *     through a mutex, /root/reference/tools/qpack-server.cpp:31).  Each model owns one HIP stream on the current device.
 *   - Weights are copied into HBM by qph_create / qph_load; the caller's buffers (or the mmap) may be released afterwards.
 *   - A call that fails because a decode attention merge timed out (its message says so) leaves the position at the
 *     last point the model verified clean: the start of that call, or earlier when state-only steps (want = 0, which
 *     do not wait for the device) ran since the last wait.  qph_pos() tells where; the cache from there on is invalid.
 */
#ifndef QPACK_HIP_H
#define QPACK_HIP_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct qph_model qph_model;

/* tensor kinds (the QPACK2 kinds the Llama path reads, /root/reference/QPACK2.md table; the kinds LlamaCuda uploads,
 * src/model_llama_cuda.cu:549-556) */
enum { QPH_F32 = 0, QPH_Q8 = 1, QPH_Q4 = 2, QPH_Q1 = 3 };

/* Model config: the config.json keys read by the reference (/root/reference/src/model_llama.cpp:21-27). */
typedef struct {
  int hidden, layers, heads, kv_heads, head_dim, ffn, vocab;
  int tied;       /* tie_embeddings: the output head is `embed` */
  int qkv_bias;   /* bq / bk / bv present */
  int max_pos;    /* max_position_embeddings */
  float rms_eps;
  double rope_theta;
} qph_config;

/* One tensor with the canonical name (/root/reference/python/qpack/convert_llama.py:5-11):
 * q8: data int8 [rows, cols], scale f32 [rows];  q4: data u8 [rows, cols/2], scale fp16 [rows, cols/32];
 * q1: data sign bits u8 [rows, cols/8] (bit c of a row's group g of 16 bytes = column 128g + c, 1 = +1), scale fp16
 * [rows, cols/128], cols a multiple of 128 (as LlamaCuda requires);  f32: data only.
 * data_coded / scale_coded: 0 for plain bytes; > 0 when the pointer holds a QPACK3 rANS blob of that many bytes
 * (/root/reference/include/qpack/rans.h, QPACK2.md:30-51), which the model decodes in HBM (the reference Container
 * decodes such blobs on the CPU at load, src/container.cpp:94-121). */
typedef struct {
  const char *name;
  int kind;
  int64_t rows, cols;
  const void *data;
  const void *scale;
  int64_t data_coded, scale_coded;
} qph_tensor;

const char *qph_last_error(void);
/* number of visible HIP devices (0 on a machine without a GPU) */
int qph_device_count(int *n);

/* ---- construction (LlamaCuda::LlamaCuda, model_llama_cuda.cu:447-484; make_llama_cuda, qpack.h:175) */
/* max_ctx <= 0 picks min(4096, max_pos) like the reference (model_llama.cpp:27). */
int qph_create(const qph_config *cfg, const qph_tensor *tensors, int n_tensors, int max_ctx, qph_model **out);
/* load_model(path, max_ctx) for arch "llama" (model_llama.cpp:221-235): mmap a QPACK1/QPACK2/QPACK3 file, read
 * config.json and the manifest, upload to HBM; QPACK3's coded blobs are uploaded coded and decoded on the GPU */
int qph_load(const char *path, int max_ctx, qph_model **out);
/* the QPACK3 decode of the model's load: coded planes, coded / raw bytes, HIP-event times of the upload (first copy
 * to last), of the decode (first launch to last; the launches run under the upload, one per upload round) and of both,
 * and the number of upload rounds (zeros for a plain file) */
typedef struct {
  int planes;
  int64_t coded_bytes, raw_bytes;
  float upload_ms, decode_ms;
  float total_ms;
  int rounds;
} qph_load_stats;
int qph_load_stats_of(const qph_model *m, qph_load_stats *out);
void qph_destroy(qph_model *m);   /* ~LlamaCuda */

/* ---- qp::Model queries (qpack.h:131-134, :164) */
int qph_vocab(const qph_model *m);
int qph_hidden(const qph_model *m);
int qph_max_ctx(const qph_model *m);
int qph_pos(const qph_model *m);
int qph_config_of(const qph_model *m, qph_config *out);

/* ---- token loop */
/* Model::step (qpack.h:136): want 0 = state only, 1 = logits (vocab floats into out), 2 = final normed hidden state
 * (hidden floats into out).  Errors: token out of range, context full (model_llama.cpp:169-170). */
int qph_step(qph_model *m, int token, int want, float *out);
/* Model::prefill (qpack.h:138): n prompt tokens, `want` applies to the last one */
int qph_prefill(qph_model *m, const int *tokens, int n, int want, float *out);
/* Model::greedy_run (qpack.h:143): out[i] = argmax after feeding token i; token i+1 = out[i].  Runs on the device with
 * no host round trip per token; returns the number of tokens produced in *produced (fewer when the context fills). */
int qph_greedy_run(qph_model *m, int token, int n, int *out, int *produced);
/* Model::prefill_all (qpack.h:152): logits of every position, n x vocab floats */
int qph_prefill_all(qph_model *m, const int *tokens, int n, float *logits);
/* Model::step / prefill with the logits kept on the device: the M largest (index, value) pairs of the last token's
 * logits, value descending and the lower index first among equal values - what the sampler's top_m and sort compute
 * from a logits vector (/root/reference/src/sampler.cpp:12-27, :41-42), here without copying the vocab floats to the
 * host.  1 <= M <= min(512, vocab); a caller wanting more candidates takes the logits (want = 1) instead. */
int qph_step_topk(qph_model *m, int token, int M, int *idx, float *val);
int qph_prefill_topk(qph_model *m, const int *tokens, int n, int M, int *idx, float *val);
/* Model::reset (qpack.h:150) */
int qph_reset(qph_model *m);
/* Model::rewind (qpack.h:160): keep the first pos tokens (0 <= pos <= current); *ok = 0 when pos is out of range */
int qph_rewind(qph_model *m, int pos, int *ok);
/* Model::checkpoint / rollback (qpack.h:157-158, model_llama.cpp:47-48): the position alone */
int qph_set_pos(qph_model *m, int pos);
/* Model::snapshot / restore (qpack.h:162-163) in the reference layout (model_llama.cpp:55-63): int32 pos, then per layer
 * the first pos rows of the fp16 K cache followed by the first pos rows of the fp16 V cache.  qph_snapshot_size gives the
 * byte count for the current position. */
int qph_snapshot_size(const qph_model *m, int64_t *bytes);
int qph_snapshot(qph_model *m, uint8_t *buf, int64_t cap);
int qph_restore(qph_model *m, const uint8_t *buf, int64_t n);

/* ---- arithmetic order (no reference counterpart: the reference has one CPU order).  mode 0 (default): this library's
 * kernels, logits within the reference's tolerance and exact int32 accumulators; mode 1: every floating-point operation
 * in the reference CPU path's order (kernels_x86.cpp, kernels.cpp:184-189, model_llama.cpp:66-201), so logits, caches
 * and greedy streams are bit-identical to qp::Llama's; slower (a verification mode).  Takes every layer kind (q8, q4,
 * q1) and a q8 or q4 output head.  Takes effect for the next call; the cache contents are kept. */
int qph_set_order(qph_model *m, int mode);

/* ---- measurement (no reference counterpart: qpack-bench times with the host clock, tools/qpack-bench.cpp:40-47) */
/* Runs n greedy decode steps from token/position as greedy_run does and reports the HIP-event time of the whole run
 * on the model's stream (*ms). */
int qph_time_greedy(qph_model *m, int token, int n, float *ms);
/* Launches one decode-step kernel `iters` times on the model's stream, walking the layers in turn as the token loop
 * does, and reports its mean HIP-event duration and its algorithmic HBM bytes per launch (mean over the layers).
 * which: 0 = fused RMSNorm + gate/up + SwiGLU matvec, 1 = down matvec, 2 = fused RMSNorm + qkv matvec, 3 = wo matvec,
 * 4 = output head matvec + argmax partials, 5 = attention at the current position. */
int qph_time_kernel(qph_model *m, int which, int iters, float *ms, double *bytes);
/* A plain device-to-device copy of `bytes` (a multiple of 16) through the kernel k_copy, `iters` times on a stream of
 * its own, with the buffers allocated and freed inside; *ms = mean HIP-event duration.  Calibrates hardware byte
 * counters (a profiler's FETCH_SIZE / WRITE_SIZE of k_copy should read `bytes` each). */
int qph_time_copy(int64_t bytes, int iters, float *ms);

/* ---- parity hooks (no reference counterpart; the int32 contract of rows_q8 / rows_q4, kernels_x86.cpp:55-106) */
/* Runs the product's matvec kernel on one matrix (host buffers in, host buffers out): activation quantisation of x,
 * y[rows] = W x, and, when sums != NULL, the exact int32 accumulators: q8 one per (row, 128-column block)
 * [rows, cols/128], q4 one per (row, 32-column group) [rows, cols/32], q1 one per (row, 128-column group)
 * [rows, cols/128] (rows_q1, kernels_x86.cpp:167-203).  xq / bs (optional) receive the int16 activations
 * and the per-block scales the kernel used. */
int qph_kernel_matvec(int kind, const void *q, const void *scale, int rows, int cols, const float *x, float *y,
                      int32_t *sums, int16_t *xq, float *bs);
/* Runs the product's batched prefill kernels on one matrix (host buffers; q and scale as in qph_kernel_matvec): each
 * row of X[B, cols] quantised as the decode step quantises it, then Y[B, rows] = X W^T on the int8 matrix cores
 * (matmul / mm_q8 / mm_q4, kernels.cpp:97-143, kernels_x86.cpp:287-371).  q8 rows use rows_q8's float epilogue per
 * token, so every Y row equals qph_kernel_matvec on that x; q4 rows have exact int32 group sums and their own fp32 order. */
int qph_kernel_matmul(int kind, const void *q, const void *scale, int rows, int cols, const float *X, int B, float *Y);

/* The reference-order products of qph_set_order(1) on one matrix: every vector of the first B - B % 4 in the lane
 * order of mm_q8 / mm_q4 (kernels_x86.cpp:287-371), the others (and B == 1) in rows_q8 / rows_q4 order; q1 (sign bits,
 * fp16 scale per 128 columns) in row_q1_nt's order for every vector (kernels_x86.cpp:163-211); bit-identical to the
 * reference's matmul() of the B vectors (kernels.cpp:97-143) without ExactBatches. */
int qph_kernel_matmul_ref(int kind, const void *q, const void *scale, int rows, int cols, const float *X, int B, float *Y);
/* The top-M selection of qph_step_topk on a host vector x[n] (parity hook; 1 <= M <= min(512, n)). */
int qph_kernel_topk(const float *x, int n, int M, int *idx, float *val);
/* No counterpart in the reference.  For callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the top-M of qph_kernel_topk on DEVICE buffers x[n] -> idx[M] / val[M],
 * enqueued on `stream` (a hipStream_t; NULL = the null stream) and not waited for.  Allocates nothing: its scratch keys
 * live in a fixed 512 KiB device array per GPU (hence n <= 262144; larger n is an error).  Calls that overlap on one
 * GPU share that array and race. */
int qph_topk_noalloc(const float *x, int n, int M, int *idx, float *val, void *stream);
/* rans::decode (/root/reference/include/qpack/rans.h:101-113) of one plain or chunked blob on the GPU: blob[len] (host)
 * -> out[cap] (host, at least the blob's raw length, which *raw receives).  Errors carry the reference's messages
 * (truncated / bad frequency table / unknown codec / stream overrun).  *ms (optional) = the decode kernel's HIP-event
 * duration. */
int qph_kernel_rans_decode(const uint8_t *blob, int64_t len, uint8_t *out, int64_t cap, int64_t *raw, float *ms);
/* qpack-pack in out (/root/reference/tools/qpack-pack.cpp, all classes): a QPACK2 file -> QPACK3, each q4 / q8 / scale /
 * f16 / f32 blob rANS-coded (16 MiB chunks above 32 MiB) where that makes it smaller; *coded = blobs coded.  Host only
 * (the writer of the coded files the loader decodes on the GPU). */
int qph_pack(const char *src, const char *dst, int threads, int *coded);

/* ---- synthetic models (no reference counterpart: the reference's files come from convert_llama.py / qpack-quantize).
 * Writes a seeded random-init Llama-family QPACK2 file; see qpack_amd/csrc/host/synth.cpp for the exact rules. */
typedef struct {
  int hidden, layers, heads, kv_heads, head_dim, ffn, vocab;
  int tied, qkv_bias, max_pos;
  int q4;        /* 0: every matrix q8; 1: layer matrices q4 (groups of 32), embed / head q8 */
  int q4m_alt;   /* with q4: wv and the w_down of even layers stay q8 */
  float rms_eps;
  double rope_theta;
  float std;     /* weight standard deviation (0.02) */
  uint64_t seed;
  char model_type[32];
  int more_bits; /* with q4 or mlp_q1: qpack-quantize's q4m / q1m policy (tools/qpack-quantize.cpp:67-74): wv and the
                    w_down of the first and last eighth of the layers and of every third layer in between stay q8 */
  int q4_head;   /* with q4: embed and lm_head q4 too (qpack-quantize --q4-head) */
  int mlp_q1;    /* w_gate / w_up / w_down in q1 (sign bits, groups of 128, scale = fp16(mean |w|)), as qpack-quantize
                    --type q1 writes them (:80-85); needs hidden and ffn multiples of 128 */
} qph_synth_spec;
int qph_synth_write(const qph_synth_spec *spec, const char *path, int threads);

#ifdef __cplusplus
}
#endif
#endif /* QPACK_HIP_H */
