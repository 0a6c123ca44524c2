// extern "C" entry points of libqpack_hip.so (declared in include/qpack_hip.h).  Each one catches every C++ exception
// and turns it into status -1 plus a thread-local message, so no exception crosses the C boundary.
#include <hip/hip_runtime.h>

#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/qpack_hip.h"
#include "hip/launch.hpp"
#include "hip/model.hpp"
#include "host/container.hpp"
#include "host/rans.hpp"
#include "host/synth.hpp"

struct qph_model {
  std::unique_ptr<qph::HipLlama> m;
};

static thread_local std::string g_err;

#define QPH_API_TRY(...)                  \
  try {                                   \
    __VA_ARGS__;                          \
    return 0;                             \
  } catch (std::exception & e) {          \
    g_err = e.what();                     \
    return -1;                            \
  } catch (...) {                         \
    g_err = "unknown C++ exception";      \
    return -1;                            \
  }

static void need(const void *p, const char *what) {
  if (!p) throw std::invalid_argument(std::string(what) + " is NULL");
}
static void hck(hipError_t e, const char *what) {
  if (e != hipSuccess) throw std::runtime_error(std::string("hip: ") + hipGetErrorString(e) + " (" + what + ")");
}

extern "C" {

const char *qph_last_error(void) { return g_err.c_str(); }

int qph_device_count(int *n) {
  QPH_API_TRY({
    need(n, "n"); int c = 0;
    if (hipGetDeviceCount(&c) != hipSuccess) c = 0;
    *n = c;
  });
}

int qph_create(const qph_config *cfg, const qph_tensor *tensors, int n_tensors, int max_ctx, qph_model **out) {
  QPH_API_TRY({
    need(cfg, "cfg"); need(tensors, "tensors"); need(out, "out");
    *out = nullptr;
    auto *h = new qph_model;
    try { h->m.reset(new qph::HipLlama(*cfg, tensors, n_tensors, max_ctx)); } catch (...) { delete h; throw; }
    *out = h;
  });
}

int qph_load(const char *path, int max_ctx, qph_model **out) {
  QPH_API_TRY({
    need(path, "path"); need(out, "out");
    *out = nullptr;
    qph::Container c(path);
    const qph::JNode &j = c.config();
    if (j.get("arch").text() != "llama") throw std::runtime_error(std::string(path) + ": arch '" + j.get("arch").text() + "' is not a Llama-family model");
    qph_config cfg{};
    cfg.hidden = (int)j.get("hidden_size").int_or(0); cfg.layers = (int)j.get("num_hidden_layers").int_or(0);
    cfg.heads = (int)j.get("num_attention_heads").int_or(0); cfg.kv_heads = (int)j.get("num_key_value_heads").int_or(0);
    cfg.head_dim = (int)j.get("head_dim").int_or(cfg.heads > 0 ? cfg.hidden / cfg.heads : 0);
    cfg.ffn = (int)j.get("intermediate_size").int_or(0); cfg.vocab = (int)j.get("vocab_size").int_or(0);
    cfg.rms_eps = (float)j.get("rms_norm_eps").num_or(1e-6); cfg.rope_theta = j.get("rope_theta").num_or(10000);
    cfg.tied = j.get("tie_embeddings").bool_or(false) ? 1 : 0;
    cfg.max_pos = (int)j.get("max_position_embeddings").int_or(1 << 20);
    std::vector<qph_tensor> ts;
    for (const qph::JNode &e : c.manifest().get("tensors").items()) {
      const qph::TensorView &t = c.at(e.get("name").text());
      if (t.kind == qph::Kind::F16) continue;   // 2-D f16 matrices are not on the HIP path; a required one is reported missing
      qph_tensor q{}; q.name = t.name.c_str(); q.data = t.data; q.scale = t.scale;
      if (t.shape.size() == 1) { q.rows = t.shape[0]; q.cols = 1; } else { q.rows = t.rows(); q.cols = t.cols(); }
      q.kind = t.kind == qph::Kind::Q8 ? QPH_Q8 : t.kind == qph::Kind::Q4 ? QPH_Q4 : t.kind == qph::Kind::Q1 ? QPH_Q1 : QPH_F32;
      q.data_coded = (int64_t)t.data_coded; q.scale_coded = (int64_t)t.scale_coded;
      ts.push_back(q);
    }
    cfg.qkv_bias = c.get("layers.0.bq") ? 1 : 0;
    auto *h = new qph_model;
    try { h->m.reset(new qph::HipLlama(cfg, ts.data(), (int)ts.size(), max_ctx)); } catch (...) { delete h; throw; }
    *out = h;
  });
}

void qph_destroy(qph_model *m) { delete m; }

int qph_load_stats_of(const qph_model *m, qph_load_stats *out) {
  QPH_API_TRY({
    need(m, "model"); need(out, "out");
    const qph::RansTiming &t = m->m->load_timing();
    out->planes = t.planes; out->coded_bytes = (int64_t)t.coded; out->raw_bytes = (int64_t)t.raw;
    out->upload_ms = t.upload_ms; out->decode_ms = t.decode_ms; out->total_ms = t.total_ms; out->rounds = t.rounds;
  });
}

int qph_vocab(const qph_model *m) { return m ? m->m->config().vocab : -1; }
int qph_hidden(const qph_model *m) { return m ? m->m->config().hidden : -1; }
int qph_max_ctx(const qph_model *m) { return m ? m->m->max_ctx() : -1; }
int qph_pos(const qph_model *m) { return m ? m->m->pos() : -1; }
int qph_config_of(const qph_model *m, qph_config *out) { QPH_API_TRY({ need(m, "model"); need(out, "out"); *out = m->m->config(); }); }

int qph_step(qph_model *m, int token, int want, float *out) {
  QPH_API_TRY({
    need(m, "model");
    if (want < 0 || want > 2) throw std::invalid_argument("want must be 0, 1 or 2");
    if (want) need(out, "out");
    m->m->step(token, want, out);
  });
}
int qph_prefill(qph_model *m, const int *tokens, int n, int want, float *out) {
  QPH_API_TRY({
    need(m, "model"); need(tokens, "tokens");
    if (want < 0 || want > 2) throw std::invalid_argument("want must be 0, 1 or 2");
    if (want) need(out, "out");
    m->m->prefill(tokens, n, want, out);
  });
}
int qph_greedy_run(qph_model *m, int token, int n, int *out, int *produced) {
  QPH_API_TRY({
    need(m, "model"); need(out, "out");
    const int r = m->m->greedy_run(token, n, out);
    if (produced) *produced = r;
  });
}
int qph_prefill_all(qph_model *m, const int *tokens, int n, float *logits) {
  QPH_API_TRY({ need(m, "model"); need(tokens, "tokens"); need(logits, "logits"); m->m->prefill_all(tokens, n, logits); });
}
int qph_step_topk(qph_model *m, int token, int M, int *idx, float *val) {
  QPH_API_TRY({ need(m, "model"); need(idx, "idx"); need(val, "val"); m->m->step_topk(token, M, idx, val); });
}
int qph_prefill_topk(qph_model *m, const int *tokens, int n, int M, int *idx, float *val) {
  QPH_API_TRY({
    need(m, "model"); need(tokens, "tokens"); need(idx, "idx"); need(val, "val");
    m->m->prefill_topk(tokens, n, M, idx, val);
  });
}
int qph_reset(qph_model *m) { QPH_API_TRY({ need(m, "model"); m->m->reset(); }); }
int qph_rewind(qph_model *m, int pos, int *ok) {
  QPH_API_TRY({ need(m, "model"); const bool r = m->m->rewind(pos); if (ok) *ok = r ? 1 : 0; });
}
int qph_set_pos(qph_model *m, int pos) { QPH_API_TRY({ need(m, "model"); m->m->set_pos(pos); }); }
int qph_snapshot_size(const qph_model *m, int64_t *bytes) { QPH_API_TRY({ need(m, "model"); need(bytes, "bytes"); *bytes = m->m->snapshot_size(); }); }
int qph_snapshot(qph_model *m, uint8_t *buf, int64_t cap) { QPH_API_TRY({ need(m, "model"); need(buf, "buf"); m->m->snapshot(buf, cap); }); }
int qph_restore(qph_model *m, const uint8_t *buf, int64_t n) { QPH_API_TRY({ need(m, "model"); need(buf, "buf"); m->m->restore(buf, n); }); }

int qph_set_order(qph_model *m, int mode) { QPH_API_TRY({ need(m, "model"); m->m->set_order(mode); }); }

int qph_time_greedy(qph_model *m, int token, int n, float *ms) {
  QPH_API_TRY({ need(m, "model"); need(ms, "ms"); *ms = m->m->time_greedy(token, n); });
}
int qph_time_kernel(qph_model *m, int which, int iters, float *ms, double *bytes) {
  QPH_API_TRY({ need(m, "model"); need(ms, "ms"); need(bytes, "bytes"); *ms = m->m->time_kernel(which, iters, bytes); });
}

int qph_time_copy(int64_t bytes, int iters, float *ms) {
  QPH_API_TRY({
    need(ms, "ms");
    if (bytes <= 0 || bytes % 16) throw std::invalid_argument("time_copy: bytes must be a positive multiple of 16");
    if (iters <= 0) iters = 1;
    void *src = nullptr, *dst = nullptr;
    hipStream_t st = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    auto cleanup = [&]() {
      if (e0) (void)hipEventDestroy(e0);
      if (e1) (void)hipEventDestroy(e1);
      if (st) (void)hipStreamDestroy(st);
      if (src) (void)hipFree(src);
      if (dst) (void)hipFree(dst);
    };
    try {
      QPH_CK(hipMalloc(&src, bytes)); QPH_CK(hipMalloc(&dst, bytes));
      QPH_CK(hipStreamCreateWithFlags(&st, hipStreamNonBlocking));
      QPH_CK(hipMemsetAsync(src, 1, bytes, st));
      QPH_CK(hipEventCreate(&e0)); QPH_CK(hipEventCreate(&e1));
      QPH_CK(qph::launch_copy(src, dst, bytes / 16, st));   // warm-up
      QPH_CK(hipEventRecord(e0, st));
      for (int i = 0; i < iters; i++) QPH_CK(qph::launch_copy(src, dst, bytes / 16, st));
      QPH_CK(hipEventRecord(e1, st));
      QPH_CK(hipEventSynchronize(e1));
      QPH_CK(hipEventElapsedTime(ms, e0, e1));
      *ms /= iters;
    } catch (...) { cleanup(); throw; }
    cleanup();
  });
}

int qph_kernel_matvec(int kind, const void *q, const void *scale, int rows, int cols, const float *x, float *y,
                      int32_t *sums, int16_t *xq, float *bs) {
  QPH_API_TRY({
    need(q, "q"); need(scale, "scale"); need(x, "x"); need(y, "y");
    if (rows <= 0 || cols <= 0 || cols % 128) throw std::invalid_argument("matvec: rows > 0 and cols a positive multiple of 128 required");
    if (kind != QPH_Q8 && kind != QPH_Q4 && kind != QPH_Q1) throw std::invalid_argument("matvec: kind must be QPH_Q8, QPH_Q4 or QPH_Q1");
    const size_t qb = kind == QPH_Q8 ? (size_t)rows * cols : kind == QPH_Q4 ? (size_t)rows * cols / 2 : (size_t)rows * cols / 8;
    const size_t sb = kind == QPH_Q8 ? 4ull * rows : kind == QPH_Q4 ? 2ull * rows * (cols / 32) : 2ull * rows * (cols / 128);
    const size_t nsum = kind == QPH_Q4 ? (size_t)rows * (cols / 32) : (size_t)rows * (cols / 128);
    std::vector<void *> bufs;
    auto alloc = [&](size_t n) { void *p = nullptr; hck(hipMalloc(&p, n), "hipMalloc"); bufs.push_back(p); return p; };
    try {
      void *dq = alloc(qb), *ds = alloc(sb); float *dx = (float *)alloc(4ull * cols), *dy = (float *)alloc(4ull * rows);
      int32_t *dsum = sums ? (int32_t *)alloc(4 * nsum) : nullptr;
      int16_t *dxq = xq ? (int16_t *)alloc(2ull * cols) : nullptr;
      float *dbs = bs ? (float *)alloc(4ull * (cols / 128)) : nullptr;
      hck(hipMemcpy(dq, q, qb, hipMemcpyHostToDevice), "upload q");
      hck(hipMemcpy(ds, scale, sb, hipMemcpyHostToDevice), "upload scale");
      hck(hipMemcpy(dx, x, 4ull * cols, hipMemcpyHostToDevice), "upload x");
      qph::MvArgs a{}; a.m[0].q = dq; a.m[0].s = ds; a.m[0].rows = rows; a.m[0].cols = cols; a.m[0].kind = kind == QPH_Q8 ? qph::MK_Q8 : kind == QPH_Q4 ? qph::MK_Q4 : qph::MK_Q1;
      a.nseg = 1; a.x = dx; a.out[0] = dy; a.dbg_sums = dsum; a.dbg_xq = dxq; a.dbg_bs = dbs;
      qph::mv_plan(a, qph::EPI_STORE);
      hck(qph::launch_matvec(qph::PRO_QUANT, qph::EPI_STORE, a, 256, nullptr), "launch matvec");
      hck(hipDeviceSynchronize(), "matvec");
      hck(hipMemcpy(y, dy, 4ull * rows, hipMemcpyDeviceToHost), "download y");
      if (sums) hck(hipMemcpy(sums, dsum, 4 * nsum, hipMemcpyDeviceToHost), "download sums");
      if (xq) hck(hipMemcpy(xq, dxq, 2ull * cols, hipMemcpyDeviceToHost), "download xq");
      if (bs) hck(hipMemcpy(bs, dbs, 4ull * (cols / 128), hipMemcpyDeviceToHost), "download bs");
    } catch (...) { for (void *p : bufs) (void)hipFree(p); throw; }
    for (void *p : bufs) (void)hipFree(p);
  });
}

int qph_kernel_topk(const float *x, int n, int M, int *idx, float *val) {
  QPH_API_TRY({
    need(x, "x"); need(idx, "idx"); need(val, "val");
    if (n <= 0 || M < 1 || M > qph::kTopkMax || M > n) throw std::invalid_argument("topk: 1 <= M <= min(512, n) required");
    std::vector<void *> bufs;
    auto alloc = [&](size_t b) { void *p = nullptr; hck(hipMalloc(&p, b), "hipMalloc"); bufs.push_back(p); return p; };
    try {
      const size_t keys = qph::topk_scratch_keys(n, M);
      float *dx = (float *)alloc(4ull * n), *dv = (float *)alloc(4ull * M);
      int *di = (int *)alloc(4ull * M);
      uint64_t *ka = (uint64_t *)alloc(8 * keys), *kb = (uint64_t *)alloc(8 * keys);
      hck(hipMemcpy(dx, x, 4ull * n, hipMemcpyHostToDevice), "upload x");
      hck(qph::launch_topk(dx, n, M, ka, kb, di, dv, nullptr), "launch topk");
      hck(hipDeviceSynchronize(), "topk");
      hck(hipMemcpy(idx, di, 4ull * M, hipMemcpyDeviceToHost), "download idx");
      hck(hipMemcpy(val, dv, 4ull * M, hipMemcpyDeviceToHost), "download val");
    } catch (...) { for (void *p : bufs) (void)hipFree(p); throw; }
    for (void *p : bufs) (void)hipFree(p);
  });
}
int qph_topk_noalloc(const float *x, int n, int M, int *idx, float *val, void *stream) {
  QPH_API_TRY({
    need(x, "x"); need(idx, "idx"); need(val, "val");
    if (n <= 0 || n > 262144) throw std::invalid_argument("topk_noalloc: n must be in [1, 262144] (the size of its fixed device buffers)");
    if (M < 1 || M > qph::kTopkMax || M > n) throw std::invalid_argument("topk_noalloc: 1 <= M <= min(512, n) required");
    hck(qph::launch_topk_noalloc(x, n, M, idx, val, (hipStream_t)stream), "launch topk");
  });
}
int qph_kernel_matmul(int kind, const void *q, const void *scale, int rows, int cols, const float *X, int B, float *Y) {
  QPH_API_TRY({
    need(q, "q"); need(scale, "scale"); need(X, "X"); need(Y, "Y");
    if (rows <= 0 || B <= 0 || cols <= 0 || cols % 128) throw std::invalid_argument("matmul: rows, B > 0 and cols a positive multiple of 128 required");
    if (kind != QPH_Q8 && kind != QPH_Q4) throw std::invalid_argument("matmul: kind must be QPH_Q8 or QPH_Q4");
    const int nb = cols / 128, G = cols / 32, ldg = (G + 3) / 4 * 4;
    const size_t qb = kind == QPH_Q8 ? (size_t)rows * cols : (size_t)rows * cols / 2;
    const size_t sb = kind == QPH_Q8 ? 4ull * rows : 2ull * rows * G;
    std::vector<void *> bufs;
    auto alloc = [&](size_t n) { void *p = nullptr; hck(hipMalloc(&p, n), "hipMalloc"); bufs.push_back(p); return p; };
    try {
      void *dq = alloc(qb), *ds = alloc(sb);
      float *dx = (float *)alloc(4ull * B * cols), *dy = (float *)alloc(4ull * B * rows), *dxb = (float *)alloc(4ull * B * nb);
      const int ldbt = (B + 63) / 64 * 64;
      float *dxbt = (float *)alloc(4ull * ldbt * nb);
      int8_t *dxh = (int8_t *)alloc((size_t)B * cols), *dxl = (int8_t *)alloc((size_t)B * cols);
      int *dxg = (int *)alloc(4ull * B * ldg);
      hck(hipMemcpy(dq, q, qb, hipMemcpyHostToDevice), "upload q");
      hck(hipMemcpy(ds, scale, sb, hipMemcpyHostToDevice), "upload scale");
      hck(hipMemcpy(dx, X, 4ull * B * cols, hipMemcpyHostToDevice), "upload X");
      qph::PfQuantArgs qa{}; qa.x = dx; qa.ldx = cols; qa.cols = cols; qa.xh = dxh; qa.xl = dxl; qa.ldq = cols; qa.xb = dxb; qa.ldb = nb;
      qa.xg = dxg; qa.ldg = ldg; qa.xbt = dxbt; qa.ldbt = ldbt;
      hck(qph::launch_pf_quant(qph::PRO_QUANT, qa, B, nullptr), "launch quant");
      qph::GemmArgs ga{}; ga.kind = kind == QPH_Q8 ? qph::MK_Q8 : qph::MK_Q4; ga.w = (const int8_t *)dq; ga.scale = (const float *)ds;
      ga.rows = rows; ga.cols = cols; ga.xh = dxh; ga.xl = dxl; ga.xb = dxb; ga.ntok = B; ga.ldq = cols; ga.ldb = nb;
      ga.xg = dxg; ga.ldg = ldg; ga.y = dy; ga.ldy = rows; ga.xbt = dxbt; ga.ldbt = ldbt;
      if (kind == QPH_Q8) {
        int *dws = (int *)alloc(4ull * qph::ws_pitch(rows) * nb);
        hck(qph::launch_rowsum_q8((const int8_t *)dq, rows, cols, dws, nullptr), "launch rowsum");
        ga.wsum = dws;
      } else {
        int *dns = (int *)alloc(4ull * rows * G); float *dsc = (float *)alloc(4ull * rows * G);
        hck(qph::launch_q4_prep((const uint8_t *)dq, (const uint16_t *)ds, rows, cols, dns, dsc, nullptr), "launch q4 prep");
        ga.q4ns = dns; ga.q4sc = dsc;
      }
      hck(qph::launch_gemm(ga, nullptr), "launch gemm");
      hck(hipDeviceSynchronize(), "matmul");
      hck(hipMemcpy(Y, dy, 4ull * B * rows, hipMemcpyDeviceToHost), "download Y");
    } catch (...) { for (void *p : bufs) (void)hipFree(p); throw; }
    for (void *p : bufs) (void)hipFree(p);
  });
}

int qph_kernel_matmul_ref(int kind, const void *q, const void *scale, int rows, int cols, const float *X, int B, float *Y) {
  QPH_API_TRY({
    need(q, "q"); need(scale, "scale"); need(X, "X"); need(Y, "Y");
    if (rows <= 0 || B <= 0 || cols <= 0 || cols % 128) throw std::invalid_argument("matmul: rows, B > 0 and cols a positive multiple of 128 required");
    if (kind != QPH_Q8 && kind != QPH_Q4 && kind != QPH_Q1) throw std::invalid_argument("matmul: kind must be QPH_Q8, QPH_Q4 or QPH_Q1");
    const int nb = cols / 128, G = cols / 32;
    const size_t qb = kind == QPH_Q8 ? (size_t)rows * cols : kind == QPH_Q4 ? (size_t)rows * cols / 2 : (size_t)rows * cols / 8;
    const size_t sb = kind == QPH_Q8 ? 4ull * rows : kind == QPH_Q4 ? 2ull * rows * G : 2ull * rows * nb;
    std::vector<void *> bufs;
    auto alloc = [&](size_t n) { void *p = nullptr; hck(hipMalloc(&p, n), "hipMalloc"); bufs.push_back(p); return p; };
    try {
      void *dq = alloc(qb), *ds = alloc(sb);
      float *dx = (float *)alloc(4ull * B * cols), *dy = (float *)alloc(4ull * B * rows), *dxb = (float *)alloc(4ull * B * nb);
      int8_t *dxh = (int8_t *)alloc((size_t)B * cols), *dxl = (int8_t *)alloc((size_t)B * cols);
      hck(hipMemcpy(dq, q, qb, hipMemcpyHostToDevice), "upload q");
      hck(hipMemcpy(ds, scale, sb, hipMemcpyHostToDevice), "upload scale");
      hck(hipMemcpy(dx, X, 4ull * B * cols, hipMemcpyHostToDevice), "upload X");
      qph::PfQuantArgs qa{}; qa.x = dx; qa.ldx = cols; qa.cols = cols; qa.xh = dxh; qa.xl = dxl; qa.ldq = cols; qa.xb = dxb; qa.ldb = nb;
      hck(qph::launch_pf_quant(qph::PRO_QUANT, qa, B, nullptr), "launch quant");
      qph::ExGemmArgs ga{}; ga.kind = kind == QPH_Q8 ? qph::MK_Q8 : kind == QPH_Q4 ? qph::MK_Q4 : qph::MK_Q1; ga.w = dq; ga.scale = (const float *)ds;
      ga.s16 = (const uint16_t *)ds; ga.rows = rows; ga.cols = cols; ga.xh = dxh; ga.xl = dxl; ga.ldq = cols; ga.xb = dxb;
      ga.ldb = nb; ga.ntok = B; ga.mm_below = B - B % 4; ga.tt = B == 1 ? 1 : 16; ga.y = dy; ga.ldy = rows;
      hck(qph::launch_ex_gemm(ga, nullptr), "launch gemm");
      hck(hipDeviceSynchronize(), "matmul");
      hck(hipMemcpy(Y, dy, 4ull * B * rows, hipMemcpyDeviceToHost), "download Y");
    } catch (...) { for (void *p : bufs) (void)hipFree(p); throw; }
    for (void *p : bufs) (void)hipFree(p);
  });
}

int qph_kernel_rans_decode(const uint8_t *blob, int64_t len, uint8_t *out, int64_t cap, int64_t *raw, float *ms) {
  QPH_API_TRY({
    need(blob, "blob"); need(out, "out");
    if (len < 0 || cap < 0) throw std::invalid_argument("rans: negative length");
    const uint64_t n = qph::rans::raw_size(blob, (size_t)len);
    if (raw) *raw = (int64_t)n;
    if ((int64_t)n > cap) throw std::invalid_argument("rans: output buffer smaller than the raw length");
    void *d = nullptr;
    hck(hipMalloc(&d, n + 16), "hipMalloc");
    try {
      qph::RansBatch b;
      qph::RansTiming tm;
      b.add(blob, (size_t)len, d, n);
      b.run(nullptr, &tm, qph::RansBatch::default_round());
      if (n) hck(hipMemcpy(out, d, n, hipMemcpyDeviceToHost), "download");
      if (ms) *ms = tm.decode_ms;
    } catch (...) { (void)hipFree(d); throw; }
    hck(hipFree(d), "hipFree");
  });
}

int qph_pack(const char *src, const char *dst, int threads, int *coded) {
  QPH_API_TRY({
    need(src, "src"); need(dst, "dst");
    const int c = qph::rans::pack(src, dst, threads);
    if (coded) *coded = c;
  });
}

int qph_synth_write(const qph_synth_spec *spec, const char *path, int threads) {
  QPH_API_TRY({ need(spec, "spec"); need(path, "path"); qph::synth_write(*spec, path, threads); });
}

}  // extern "C"
