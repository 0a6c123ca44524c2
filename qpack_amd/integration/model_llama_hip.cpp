// qpack's Llama model on the MI355X: the qp::Model adapter over libqpack_hip.so that a qpack maintainer adds as
// src/model_llama_hip.cpp.  It replaces the CUDA model LlamaCuda / make_llama_cuda (/root/reference/include/qpack/
// qpack.h:128-177, /root/reference/src/model_llama_cuda.cu) method for method through the C ABI of include/qpack_hip.h,
// and is selected in load_model (/root/reference/src/model_llama.cpp:221-235) by QPACK_DEVICE=hip.
//
// Built and linked against the reference's own headers and sources by qpack_amd/integration/Makefile (the test
// tests/test_integration.py), together with tools/qpack-bench.cpp and the check harness adapter_check.cpp.
//
// QPACK3 files: the reference's Container decodes rANS-coded blobs on the CPU when it opens the file
// (src/container.cpp:41, :94-121), and every reference caller needs that Container (config, tokenizer, file size), so
// through this adapter the model is built from decoded blobs.  The GPU decoder serves callers of the C ABI that open
// the file with qph_load and need no Container.
#include <cstdlib>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "qpack/qpack.h"
#include "qpack_hip.h"
#include "sampler_hip.hpp"

namespace qp {
namespace {

void ck(int rc) { if (rc) throw std::runtime_error(std::string("hip: ") + qph_last_error()); }

float half_value(uint16_t h) {   // IEEE binary16 -> float (f16 norm vectors, widened once at load)
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t bits;
  if (e == 31) bits = s | 0x7f800000u | (m << 13);
  else if (e) bits = s | ((e + 112u) << 23) | (m << 13);
  else if (!m) bits = s;
  else { int k = 0; uint32_t mm = m; while (!(mm & 1024u)) { mm <<= 1; k++; } bits = s | ((uint32_t)(113 - k) << 23) | ((mm & 1023u) << 13); }
  float f; memcpy(&f, &bits, 4); return f;
}

class LlamaHip : public Model {
 public:
  // a model built from an open Container: its tensors, as they lie in the mmap, are copied to HBM by qph_create
  LlamaHip(std::shared_ptr<Container> c, int max_ctx) {
    c_ = c; cfg_ = c->config();
    // the config keys Llama reads (model_llama.cpp:21-27)
    qph_config k{};
    k.hidden = (int)cfg_["hidden_size"].as_int(); k.layers = (int)cfg_["num_hidden_layers"].as_int();
    k.heads = (int)cfg_["num_attention_heads"].as_int(); k.kv_heads = (int)cfg_["num_key_value_heads"].as_int();
    k.head_dim = (int)cfg_["head_dim"].as_int(k.heads ? k.hidden / k.heads : 0); k.ffn = (int)cfg_["intermediate_size"].as_int();
    k.vocab = (int)cfg_["vocab_size"].as_int(); k.rms_eps = (float)cfg_["rms_norm_eps"].as_num(1e-6);
    k.rope_theta = cfg_["rope_theta"].as_num(10000); k.tied = cfg_["tie_embeddings"].as_bool(false) ? 1 : 0;
    k.max_pos = (int)cfg_["max_position_embeddings"].as_int(1 << 20); k.qkv_bias = c->get("layers.0.bq") ? 1 : 0;
    std::vector<qph_tensor> ts;
    std::vector<std::vector<float>> widened;
    ts.reserve(c->tensors().size());
    widened.reserve(c->tensors().size());
    for (auto &kv : c->tensors()) {
      const Tensor &t = kv.second;
      qph_tensor q{};
      q.name = kv.first.c_str(); q.rows = t.rows(); q.cols = t.shape.size() == 1 ? 1 : t.cols(); q.data = t.data;
      q.data_coded = 0; q.scale_coded = 0;   // the reference Container has decoded QPACK3 blobs already
      if (t.kind == Kind::Q8) { q.kind = QPH_Q8; q.scale = t.scale; }
      else if (t.kind == Kind::Q4) { q.kind = QPH_Q4; q.scale = t.scale16; }
      else if (t.kind == Kind::Q1) { q.kind = QPH_Q1; q.scale = t.scale16; }
      else if (t.kind == Kind::F32) { q.kind = QPH_F32; q.scale = nullptr; }
      else if (t.kind == Kind::F16 && t.shape.size() == 1) {   // norm / bias vectors stored as f16
        std::vector<float> w((size_t)t.numel());
        for (size_t i = 0; i < w.size(); i++) w[i] = half_value(((const uint16_t *)t.data)[i]);
        widened.push_back(std::move(w));
        q.kind = QPH_F32; q.data = widened.back().data(); q.scale = nullptr;
      } else continue;   // kinds the Llama token loop never reads
      ts.push_back(q);
    }
    ck(qph_create(&k, ts.data(), (int)ts.size(), max_ctx, &m_));   // copies to HBM: `widened` may go afterwards
    // QPACK_HIP_ORDER=reference: the reference CPU path's float order (logits bit-identical to make_llama's); the
    // default order is the fast kernels', within the logit tolerance
    if (const char *o = getenv("QPACK_HIP_ORDER")) {
      if (!strcmp(o, "reference")) ck(qph_set_order(m_, 1));
      else if (strcmp(o, "default")) { qph_destroy(m_); throw std::runtime_error("QPACK_HIP_ORDER: 'default' or 'reference'"); }
    }
    out_.resize((size_t)std::max(qph_vocab(m_), qph_hidden(m_)));
  }
  ~LlamaHip() override { qph_destroy(m_); }

  int vocab() const override { return qph_vocab(m_); }
  int hidden() const override { return qph_hidden(m_); }
  int max_ctx() const override { return qph_max_ctx(m_); }
  int pos() const override { return qph_pos(m_); }
  // the returned pointer stays valid until the next call (LlamaCuda's pinned buffer behaves the same)
  const float *step(int token, int want) override {
    ck(qph_step(m_, token, want, want ? out_.data() : nullptr));
    return want ? out_.data() : nullptr;
  }
  const float *prefill(const int *tokens, int n, int want) override {
    ck(qph_prefill(m_, tokens, n, want, want ? out_.data() : nullptr));
    return want ? out_.data() : nullptr;
  }
  int greedy_run(int token, int n, int *out) override { int got = 0; ck(qph_greedy_run(m_, token, n, out, &got)); return got; }
  void prefill_all(const int *tokens, int n, float *logits) override { ck(qph_prefill_all(m_, tokens, n, logits)); }
  void reset() override { ck(qph_reset(m_)); }
  bool rewind(int p) override { int ok = 0; ck(qph_rewind(m_, p, &ok)); return ok != 0; }
  std::vector<uint8_t> checkpoint() const override {   // the position alone, as Llama (model_llama.cpp:47-48)
    std::vector<uint8_t> b(4); const int p = qph_pos(m_); memcpy(b.data(), &p, 4); return b;
  }
  void rollback(const std::vector<uint8_t> &c) override { int p; memcpy(&p, c.data(), 4); ck(qph_set_pos(m_, p)); }
  std::vector<uint8_t> snapshot() const override {    // the bytes of Llama::snapshot (model_llama.cpp:55-63)
    int64_t n = 0; ck(qph_snapshot_size(m_, &n));
    std::vector<uint8_t> b((size_t)n); ck(qph_snapshot(m_, b.data(), n)); return b;
  }
  void restore(const std::vector<uint8_t> &s) override { ck(qph_restore(m_, s.data(), (int64_t)s.size())); }
  // the reference's CUDA model marks its backend the same way (model_llama_cuda.cu:500)
  std::string arch() const override { return "llama:" + cfg_["model_type"].as_str() + "@hip"; }

  // the device top-M of the next logits (qph_step_topk): the candidates Sampler::dist would take from top_m
  void step_topk(int token, int M, std::vector<std::pair<int, float>> &cand) {
    std::vector<int> idx((size_t)M);
    std::vector<float> val((size_t)M);
    ck(qph_step_topk(m_, token, M, idx.data(), val.data()));
    cand.resize((size_t)M);
    for (int i = 0; i < M; i++) cand[(size_t)i] = {idx[(size_t)i], val[(size_t)i]};
  }

 private:
  qph_model *m_ = nullptr;
  std::vector<float> out_;
};

}  // namespace

std::unique_ptr<Model> make_llama_hip(std::shared_ptr<Container> c, int max_ctx) {
  return std::unique_ptr<Model>(new LlamaHip(std::move(c), max_ctx));
}

bool hip_step_candidates(Model &m, int token, int M, std::vector<std::pair<int, float>> &cand) {
  LlamaHip *h = dynamic_cast<LlamaHip *>(&m);
  if (!h) return false;
  h->step_topk(token, M, cand);
  return true;
}

}  // namespace qp
