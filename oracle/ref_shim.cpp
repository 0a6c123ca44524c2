// C-ABI harness over the reference qpack CPU engine, compiled from the reference's own sources by oracle/Makefile into
// oracle/_ref/libqpref.so.  TEST INFRASTRUCTURE ONLY: tests/, tests/golden/make_golden.py and bench.py's cpu_baseline leg
// load it as the checker / CPU baseline; the product (qpack_amd/) never links or calls it.
//
// Every entry point returns 0 on success and -1 on a C++ exception (message via qpref_error()), mirroring how the
// reference reports errors (std::runtime_error everywhere, /root/reference/src/model_llama.cpp:169-170).
#include <cstdint>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "qpack/engine.h"
#include "qpack/qpack.h"
#include "qpack/rans.h"

namespace qp { namespace impl {
// row kernels of /root/reference/src/kernels_impl.h:29-30 (declared there; repeated here so the shim needs only the
// public include directory)
void rows_q8(const int8_t *Q, const float *scale, const int16_t *xq, const float *bs, float *y, int r0, int r1, int cols);
void rows_q4(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int r0, int r1, int cols);
void rows_q1(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int r0, int r1, int cols);
}}

static thread_local std::string g_err;
#define QPREF_TRY(...) try { __VA_ARGS__; return 0; } catch (std::exception &e) { g_err = e.what(); return -1; }

extern "C" {

const char *qpref_error() { return g_err.c_str(); }

// must run before anything touches qp::pool() (/root/reference/src/threads.cpp:92-99)
void qpref_set_threads(int n) { qp::set_threads(n); }
int qpref_threads() { return qp::pool().size(); }

int qpref_load(const char *path, int max_ctx, void **out) {
  QPREF_TRY(*out = qp::load_model(path, max_ctx).release());
}
void qpref_free(void *m) { delete (qp::Model *)m; }
int qpref_vocab(void *m) { return ((qp::Model *)m)->vocab(); }
int qpref_hidden(void *m) { return ((qp::Model *)m)->hidden(); }
int qpref_pos(void *m) { return ((qp::Model *)m)->pos(); }
int qpref_max_ctx(void *m) { return ((qp::Model *)m)->max_ctx(); }
void qpref_reset(void *m) { ((qp::Model *)m)->reset(); }

// want 1 copies vocab() floats, want 2 hidden() floats into out (/root/reference/include/qpack/qpack.h:136)
int qpref_step(void *mp, int tok, int want, float *out) {
  QPREF_TRY({
    qp::Model *m = (qp::Model *)mp; const float *r = m->step(tok, want);
    if (want && out && r) memcpy(out, r, 4ull * (want == 1 ? m->vocab() : m->hidden()));
  });
}
int qpref_prefill(void *mp, const int *toks, int n, int want, float *out) {
  QPREF_TRY({
    qp::Model *m = (qp::Model *)mp; const float *r = m->prefill(toks, n, want);
    if (want && out && r) memcpy(out, r, 4ull * (want == 1 ? m->vocab() : m->hidden()));
  });
}
int qpref_greedy(void *mp, int tok, int n, int *out) { QPREF_TRY(((qp::Model *)mp)->greedy_run(tok, n, out)); }
// Model::rewind (qpack.h:160): 1 when the model kept the first pos tokens
int qpref_rewind(void *mp, int pos) { return ((qp::Model *)mp)->rewind(pos) ? 1 : 0; }
// Model::prefill_all (qpack.h:152), under ExactBatches when `exact` (how Session's speculative verification calls it,
// /root/reference/src/chat.cpp:233): n x vocab logits
int qpref_prefill_all(void *mp, const int *toks, int n, float *out, int exact) {
  QPREF_TRY({
    qp::Model *m = (qp::Model *)mp;
    if (exact) { qp::ExactBatches ex; m->prefill_all(toks, n, out); }
    else m->prefill_all(toks, n, out);
  });
}
// the sampler's candidate list for top_k = M (Sampler::dist, /root/reference/src/sampler.cpp:29-57, with no penalty,
// temperature 1, top-p and min-p off): top_m, then the sort by value (lower index first among equal values); the
// indices in that order
int qpref_sampler_topk(const float *x, int V, int M, int *idx) {
  QPREF_TRY({
    qp::SamplerParams p; p.temperature = 1.f; p.top_k = M; p.top_p = 1.f; p.min_p = 0.f; p.repeat_penalty = 1.f; p.seed = 1;
    qp::Sampler s(p);
    std::vector<std::pair<int, float>> d;
    s.dist(x, V, {}, d);
    if ((int)d.size() != M) throw std::runtime_error("sampler returned " + std::to_string(d.size()) + " candidates");
    for (int i = 0; i < M; i++) idx[i] = d[i].first;
  });
}

// snapshot layout of /root/reference/src/model_llama.cpp:55-59; call with buf = nullptr to get the size
int64_t qpref_snapshot(void *mp, uint8_t *buf, int64_t cap) {
  try {
    std::vector<uint8_t> s = ((qp::Model *)mp)->snapshot();
    if (buf) { if ((int64_t)s.size() > cap) { g_err = "snapshot buffer too small"; return -1; } memcpy(buf, s.data(), s.size()); }
    return (int64_t)s.size();
  } catch (std::exception &e) { g_err = e.what(); return -1; }
}
int qpref_restore(void *mp, const uint8_t *buf, int64_t n) {
  QPREF_TRY(((qp::Model *)mp)->restore(std::vector<uint8_t>(buf, buf + n)));
}

// ---- kernel level: the public dispatch functions of /root/reference/src/kernels.cpp on caller-owned arrays
static qp::Tensor mk(int kind, const void *q, const void *s, int rows, int cols) {
  qp::Tensor t; t.name = "shim"; t.shape = {rows, cols}; t.data = q;
  if (kind == 0) { t.kind = qp::Kind::Q8; t.scale = (const float *)s; }
  else if (kind == 1) { t.kind = qp::Kind::Q4; t.scale16 = (const uint16_t *)s; t.group = 32; }
  else if (kind == 2) { t.kind = qp::Kind::F32; }
  else if (kind == 3) { t.kind = qp::Kind::Q1; t.scale16 = (const uint16_t *)s; t.group = 128; }
  else throw std::runtime_error("shim: bad kind");
  return t;
}
// kind 0 = q8, 1 = q4, 2 = f32, 3 = q1. matvec: quant_rows + rows_q8/rows_q4 (kernels.cpp:72-96)
int qpref_matvec(int kind, const void *q, const void *s, int rows, int cols, const float *x, float *y) {
  QPREF_TRY({ qp::Tensor t = mk(kind, q, s, rows, cols); qp::matvec(t, x, y, rows, cols); });
}
// matmul: B vectors (kernels.cpp:97-143); exact = 1 holds ExactBatches (row_*_multi path, B <= 16)
int qpref_matmul(int kind, const void *q, const void *s, int rows, int cols, const float *X, int B, float *Y, int exact) {
  QPREF_TRY({
    qp::Tensor t = mk(kind, q, s, rows, cols);
    if (exact) { qp::ExactBatches eb; qp::matmul(t, X, B, cols, Y, rows, rows, cols); }
    else qp::matmul(t, X, B, cols, Y, rows, rows, cols);
  });
}
// the row kernels on caller-quantised activations (kernels_x86.cpp:55-106)
void qpref_rows_q8(const int8_t *Q, const float *scale, const int16_t *xq, const float *bs, float *y, int rows, int cols) {
  qp::impl::rows_q8(Q, scale, xq, bs, y, 0, rows, cols);
}
void qpref_rows_q4(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int rows, int cols) {
  qp::impl::rows_q4(Q, S, xq, bs, y, 0, rows, cols);
}
void qpref_rows_q1(const uint8_t *Q, const uint16_t *S, const int16_t *xq, const float *bs, float *y, int rows, int cols) {
  qp::impl::rows_q1(Q, S, xq, bs, y, 0, rows, cols);
}
void qpref_rmsnorm(const float *x, const float *w, int n, float eps, float *out) { qp::rmsnorm(x, w, n, eps, out); }
void qpref_silu_mul(float *g, const float *u, int n) { qp::silu_mul(g, u, n); }
void qpref_exp_v(const float *x, float *y, int n) { qp::exp_v(x, y, n); }
void qpref_to_f16(const float *x, uint16_t *y, int n) { qp::to_f16(x, y, n); }
void qpref_row_f32(int kind, const void *q, const void *s, int rows, int cols, int r, float *out) {
  qp::Tensor t = mk(kind, q, s, rows, cols); qp::row_f32(t, r, out);
}

// QPACK3 rANS codec (include/qpack/rans.h): encode (:81-93) into out[cap]; *n_out = the blob length
int qpref_rans_encode(const uint8_t *raw, int64_t n, int codec, int planes, uint8_t *out, int64_t cap, int64_t *n_out) {
  QPREF_TRY({
    const std::vector<uint8_t> b = qp::rans::encode(raw, (size_t)n, codec, planes);
    if ((int64_t)b.size() > cap) throw std::runtime_error("qpref_rans_encode: output buffer too small");
    memcpy(out, b.data(), b.size()); *n_out = (int64_t)b.size();
  });
}
// decode (:101-113) of a plain or chunked blob; out must hold the raw size (:75)
int qpref_rans_decode(const uint8_t *p, int64_t len, uint8_t *out) { QPREF_TRY(qp::rans::decode(p, (size_t)len, out)); }
int64_t qpref_rans_raw_size(const uint8_t *p, int64_t len) {
  try { return (int64_t)qp::rans::raw_size(p, (size_t)len); } catch (std::exception &e) { g_err = e.what(); return -1; }
}

}  // extern "C"
