#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <stdexcept>

#include "../host/rans.hpp"
#include "launch.hpp"

namespace qph {

static constexpr unsigned kRing = 256;   // pinned control slots (one per host-driven step in flight)

void *HipLlama::dalloc(size_t bytes) {
  void *p = nullptr;
  QPH_CK(hipMalloc(&p, std::max<size_t>(bytes, 256)));
  allocs_.push_back(p);
  return p;
}

DMat HipLlama::upload(const qph_tensor &t) {
  DMat m{}; m.rows = (int)t.rows; m.cols = (int)t.cols;
  size_t qb = 0, sb = 0;
  if (t.kind == QPH_Q8) { m.kind = MK_Q8; qb = (size_t)t.rows * t.cols; sb = 4ull * t.rows; }
  else if (t.kind == QPH_Q4) {
    if (t.cols % 32) throw std::runtime_error(std::string("hip: q4 tensor ") + t.name + " needs cols % 32 == 0");
    m.kind = MK_Q4; qb = (size_t)t.rows * t.cols / 2; sb = 2ull * t.rows * (t.cols / 32);
  } else if (t.kind == QPH_Q1) {   // LlamaCuda's condition (model_llama_cuda.cu:554)
    if (t.cols % 128) throw std::runtime_error(std::string("hip: q1 tensor ") + t.name + " needs cols % 128 == 0");
    m.kind = MK_Q1; qb = (size_t)t.rows * t.cols / 8; sb = 2ull * t.rows * (t.cols / 128);
  } else throw std::runtime_error(std::string("hip: matrix ") + t.name + " must be q8, q4 or q1");
  if (!t.data || !t.scale) throw std::runtime_error(std::string("hip: tensor ") + t.name + " has no data");
  m.q = place(t.data, t.data_coded, qb, t.name);
  m.s = place(t.scale, t.scale_coded, sb, t.name);
  return m;
}

// a device copy of `bytes` raw bytes: copied now, or, from a rANS blob of `coded` bytes, decoded with the batch of
// coded blobs that the constructor runs once every tensor is placed (the buffer is as large as the blob's raw length
// when that is longer, as a longer plain blob would be)
void *HipLlama::place(const void *src, int64_t coded, size_t bytes, const char *name) {
  if (coded < 0) throw std::runtime_error(std::string("hip: tensor ") + name + " has a negative coded length");
  if (!coded) {
    void *p = dalloc(bytes);
    QPH_CK(hipMemcpy(p, src, bytes, hipMemcpyHostToDevice));
    return p;
  }
  const uint64_t raw = rans::raw_size((const uint8_t *)src, (size_t)coded);
  if (raw < bytes) throw std::runtime_error(std::string("hip: coded tensor ") + name + " decodes to fewer bytes than its shape needs");
  void *p = dalloc(raw);
  rans_.add((const uint8_t *)src, (size_t)coded, p, raw);
  return p;
}

const float *HipLlama::upload_f32(const qph_tensor &t, int64_t n) {
  if (t.kind != QPH_F32) throw std::runtime_error(std::string("hip: tensor ") + t.name + " must be f32");
  if (t.rows * std::max<int64_t>(t.cols, 1) != n) throw std::runtime_error(std::string("hip: tensor ") + t.name + " has the wrong size");
  return (const float *)place(t.data, t.data_coded, 4ull * n, t.name);
}

HipLlama::HipLlama(const qph_config &cfg, const qph_tensor *tensors, int n, int max_ctx) : cfg_(cfg) {
  const int d = cfg.hidden, nh = cfg.heads, nkv = cfg.kv_heads, hd = cfg.head_dim, ff = cfg.ffn, V = cfg.vocab;
  if (d <= 0 || cfg.layers <= 0 || nh <= 0 || nkv <= 0 || ff <= 0 || V <= 0) throw std::runtime_error("hip: bad model config");
  if (hd != 64 && hd != 128) throw std::runtime_error("hip: head_dim must be 64 or 128");
  if (nh % nkv || nh / nkv > 8) throw std::runtime_error("hip: unsupported GQA ratio (heads / kv_heads must be an integer <= 8)");
  qd_ = nh * hd; kvd_ = nkv * hd;
  if (d % 128 || ff % 128 || qd_ % 128) throw std::runtime_error("hip: hidden, ffn and heads * head_dim must be multiples of 128");
  const int limit = cfg.max_pos > 0 ? cfg.max_pos : (1 << 20);
  ctx_ = max_ctx > 0 ? max_ctx : std::min(4096, limit);
  std::map<std::string, const qph_tensor *> by;
  for (int i = 0; i < n; i++) by[tensors[i].name] = &tensors[i];
  auto need = [&](const std::string &nm) -> const qph_tensor & {
    auto it = by.find(nm);
    if (it == by.end()) throw std::runtime_error("hip: missing tensor " + nm);
    return *it->second;
  };
  auto opt = [&](const std::string &nm) -> const qph_tensor * { auto it = by.find(nm); return it == by.end() ? nullptr : it->second; };
  auto shape = [&](const DMat &m, int r, int c, const std::string &nm) {
    if (m.rows != r || m.cols != c) throw std::runtime_error("hip: tensor " + nm + " has an unexpected shape");
  };
  int dev = 0;
  QPH_CK(hipGetDevice(&dev));
  QPH_CK(hipDeviceGetAttribute(&cus_, hipDeviceAttributeMultiprocessorCount, dev));
  g_mv_config.cus = cus_;
  QPH_CK(hipStreamCreateWithFlags(&st_, hipStreamNonBlocking));
  embed_ = upload(need("embed")); shape(embed_, V, d, "embed");
  if (cfg.tied) head_ = embed_;
  else { head_ = upload(need("lm_head")); shape(head_, V, d, "lm_head"); }
  fnorm_ = upload_f32(need("final_norm"), d);
  for (int l = 0; l < cfg.layers; l++) {
    const std::string p = "layers." + std::to_string(l) + ".";
    Layer ly;
    ly.an = upload_f32(need(p + "attn_norm"), d); ly.fn = upload_f32(need(p + "ffn_norm"), d);
    ly.wq = upload(need(p + "wq")); shape(ly.wq, qd_, d, p + "wq");
    ly.wk = upload(need(p + "wk")); shape(ly.wk, kvd_, d, p + "wk");
    ly.wv = upload(need(p + "wv")); shape(ly.wv, kvd_, d, p + "wv");
    ly.wo = upload(need(p + "wo")); shape(ly.wo, d, qd_, p + "wo");
    ly.wg = upload(need(p + "w_gate")); shape(ly.wg, ff, d, p + "w_gate");
    ly.wu = upload(need(p + "w_up")); shape(ly.wu, ff, d, p + "w_up");
    ly.wd = upload(need(p + "w_down")); shape(ly.wd, d, ff, p + "w_down");
    if (ly.wg.kind != ly.wu.kind) throw std::runtime_error("hip: w_gate and w_up of layer " + std::to_string(l) + " must have the same kind");
    const qph_tensor *bq = opt(p + "bq");
    if (bq) { ly.bq = upload_f32(*bq, qd_); ly.bk = upload_f32(need(p + "bk"), kvd_); ly.bv = upload_f32(need(p + "bv"), kvd_); }
    layers_.push_back(ly);
  }
  rans_.run(st_, &rans_tm_, RansBatch::default_round());   // QPACK3: the coded blobs decode in HBM under their upload
  // context splits per kv group: one per 64 positions of the full context, at most 48 (the kernel activates
  // min(this, ceil(T / 64)) of them beyond one workgroup's reach).  At C5's 16K context 48 splits beat 64: fewer
  // partials for the merge launch outweigh the idle CUs (same-box greedy 546.8 -> 550.8 tok/s; 40: 538.9, 56: 548.6)
  max_chunks_ = std::max(1, std::min(48, (ctx_ + 63) / 64));
  if (const char *e = getenv("QPH_ATTN_SPLITS")) max_chunks_ = std::max(1, std::min(64, atoi(e)));
  if (const char *e = getenv("QPH_ATTN_SINGLE")) attn_single_ = std::max(0, atoi(e));
  if (const char *e = getenv("QPH_ATTN_SPLIT_POS")) attn_split_pos_ = std::max(0, atoi(e));
  // test hook: the bound of a merger's wait for the other splits (the failure path forced from the host)
  if (const char *e = getenv("QPH_ATTN_SPIN")) attn_spin_ = std::max(0, atoi(e));
  attn_force_late_ = getenv("QPH_ATTN_FORCE_LATE") != nullptr;   // test hook: the same failure without the race
  if (const char *e = getenv("QPH_MV_SPLIT")) split_chain_ = atoi(e) != 0;
  {  // long contexts: the splits' merge as a launch of its own from lm_splits_ splits (QPH_ATTN_MERGE_SEP: that
     // threshold; 0: merged in-kernel everywhere)
    const char *e = getenv("QPH_ATTN_MERGE_SEP");
    lm_splits_ = e ? std::max(0, atoi(e)) : kLongMergeSplits;
    lm_min_ = attn_long_merge_min(hd, attn_single_, attn_split_pos_, max_chunks_, lm_splits_);
    if (lm_min_ > ctx_) lm_min_ = 0;
  }

  counters_ = (int *)dalloc(8ull * nkv);
  const size_t kvn = (size_t)cfg.layers * ctx_ * kvd_;
  kc_ = (uint16_t *)dalloc(kvn * 2); vc_ = (uint16_t *)dalloc(kvn * 2);
  QPH_CK(hipMemset(kc_, 0, kvn * 2)); QPH_CK(hipMemset(vc_, 0, kvn * 2));
  x_ = (float *)dalloc(4ull * d); xn_ = (float *)dalloc(4ull * d); q_ = (float *)dalloc(4ull * qd_);
  k_ = (float *)dalloc(4ull * kvd_); v_ = (float *)dalloc(4ull * kvd_); att_ = (float *)dalloc(4ull * qd_);
  h_ = (float *)dalloc(4ull * ff); logits_ = (float *)dalloc(4ull * V);
  part_ = (float *)dalloc(4ull * nh * max_chunks_ * (hd + 2));
  q16_ = (uint16_t *)dalloc(4ull * qd_);
  QPH_CK(hipMemset(counters_, 0, 8ull * nkv));
  {  // decode attention fused with wo (q8 wo on every layer), short contexts: per kv group with the partials summed by
     // gate / up (a group's heads whole 128-column blocks), else every group in each workgroup with whole wo rows
    int rc = 0, nl = 0;
    bool ok = !layers_.empty(), rows_ok = !layers_.empty();
    for (const Layer &ly : layers_) rows_ok = rows_ok && attn_wo_rows_fits(hd, nh, nkv, ly.wo, g_mv_config.cus, &rc, &nl);
    // QPH_AWO_SUM=0: the gate / up prologue adds the group parts instead of k_attn_wo's last arrivals
    const char *es = getenv("QPH_AWO_SUM");
    awo_sum_ = !(es && atoi(es) == 0);
    for (const Layer &ly : layers_) {
      ok = ok && attn_wo_fits(hd, nh, nkv, ly.wo, g_mv_config.cus, &rc, &nl);
      if (awo_sum_) continue;
      // the gate / up launch that adds the group partials (their LDS staging must fit)
      MvArgs a{}; a.m[0] = ly.wg; a.m[1] = ly.wu; a.nseg = 2; a.part = x_; a.nparts = nkv; a.pstride = (size_t)d;
      a.plan_only = 1;
      mv_plan(a, EPI_SWIGLU);
      ok = ok && launch_matvec(PRO_NORM_SUM, EPI_SWIGLU, a, 1 << 20, st_) == hipSuccess;
    }
    const char *e = getenv("QPH_AWO_MAX");   // longest context (positions) that takes the fused kernel; 0: never
    awo_rows_ = !ok && rows_ok;
    // the rows kernel: up to the contexts where the split attention also runs one split per group (bit-identical)
    const int dflt = ok ? kAwoMaxDefault : awo_rows_ ? (attn_single_ > 0 ? attn_single_ : attn_single_max(hd)) : 0;
    awo_max_ = ok || awo_rows_ ? (e ? std::max(0, atoi(e)) : dflt) : 0;
    if (awo_max_ > 0 && !awo_rows_) {
      awo_rc_ = rc;
      awo_part_ = (float *)dalloc(4ull * nkv * d);
      xs_ = (float *)dalloc(4ull * d);
      awo_cnt_ = (int *)dalloc(4ull * rc * 8);   // [row chunk][wave]
      QPH_CK(hipMemset(awo_cnt_, 0, 4ull * rc * 8));
    }
  }
  head_grid_ = cus_ * 4;
  amax_ = (float2 *)dalloc(sizeof(float2) * head_grid_);
  {  // partials of workgroups a smaller launch does not use must never win the pick
    std::vector<float2> init((size_t)head_grid_, make_float2(-INFINITY, __builtin_bit_cast(float, 0x7fffffff)));
    QPH_CK(hipMemcpy(amax_, init.data(), init.size() * sizeof(float2), hipMemcpyHostToDevice));
  }
  ctl_ = (Ctl *)dalloc(sizeof(Ctl));
  out_tok_ = (int *)dalloc(4ull * (ctx_ + 1));
  // batched prompt path: every layer matrix q8 or q4 (the int8 MFMA products; in the default order a model with q1
  // layers takes its prompts through decode steps); chunks of up to pf_cap_ tokens.  The prompt buffers are allocated
  // either way: the reference-order prompt (k_ex_gemm, which takes q1 matrices too) uses them
  pf_ok_ = true;
  for (const Layer &ly : layers_)
    for (const DMat *m : {&ly.wq, &ly.wk, &ly.wv, &ly.wo, &ly.wg, &ly.wu, &ly.wd})
      pf_ok_ = pf_ok_ && (m->kind == MK_Q8 || m->kind == MK_Q4);
  {
    for (Layer &ly : layers_)
      for (DMat *m : {&ly.wq, &ly.wk, &ly.wv, &ly.wo, &ly.wg, &ly.wu, &ly.wd}) {
        if (!pf_ok_) break;   // the batched products' per-matrix sums: q8 / q4 models only
        if (m->kind == MK_Q8) {
          int *rs = (int *)dalloc(4ull * ws_pitch(m->rows) * (m->cols / 128));
          QPH_CK(launch_rowsum_q8((const int8_t *)m->q, m->rows, m->cols, rs, st_));
          m->rs = rs;
        } else {
          int *ns = (int *)dalloc(4ull * m->rows * (m->cols / 32));
          float *sc = (float *)dalloc(4ull * m->rows * (m->cols / 32));
          QPH_CK(launch_q4_prep((const uint8_t *)m->q, (const uint16_t *)m->s, m->rows, m->cols, ns, sc, st_));
          m->q4ns = ns; m->q4sc = sc;
        }
      }
    QPH_CK(hipStreamSynchronize(st_));
    pf_cap_ = std::min(kPfChunk, ctx_);
    if (const char *e = getenv("QPH_PF_CHUNK")) pf_cap_ = std::max(1, std::min(pf_cap_, atoi(e)));   // test hook
    const size_t B = pf_cap_, wide = std::max({d, qd_, ff});
    pf_ldq_ = (int)(wide + 15) / 16 * 16;
    pf_x_ = (float *)dalloc(4 * B * d); pf_q_ = (float *)dalloc(4 * B * qd_); pf_att_ = (float *)dalloc(4 * B * qd_);
    pf_k_ = (float *)dalloc(4 * B * kvd_); pf_v_ = (float *)dalloc(4 * B * kvd_);
    pf_g_ = (float *)dalloc(4 * B * ff);
    pf_xh_ = (int8_t *)dalloc(B * pf_ldq_); pf_xl_ = (int8_t *)dalloc(B * pf_ldq_);
    pf_xh2_ = (int8_t *)dalloc(B * pf_ldq_); pf_xl2_ = (int8_t *)dalloc(B * pf_ldq_);   // the SwiGLU output, quantised
    pf_xb_ = (float *)dalloc(4 * B * (pf_ldq_ / 128 + 1));
    pf_ldbt_ = (int)(B + 63) / 64 * 64;
    pf_xbt_ = (float *)dalloc(4ull * pf_ldbt_ * (pf_ldq_ / 128 + 1));
    pf_xb2_ = (float *)dalloc(4 * B * (pf_ldq_ / 128 + 1));
    pf_xbt2_ = (float *)dalloc(4ull * pf_ldbt_ * (pf_ldq_ / 128 + 1));
    pf_ldg_ = (pf_ldq_ / 32 + 3) / 4 * 4;
    pf_xg_ = (int *)dalloc(4 * B * pf_ldg_);
    pf_tok_ = (int *)dalloc(4 * B);
  }
  // RoPE tables in the reference's precision: inv_i = 1 / theta^(2i/hd) and angle pos * inv_i in double, cos / sin
  // rounded to float (model_llama.cpp:39, :173-175)
  const int half = hd / 2;
  std::vector<float> cs((size_t)ctx_ * half), sn((size_t)ctx_ * half);
  for (int i = 0; i < half; i++) {
    const double inv = 1.0 / std::pow(cfg.rope_theta, (2.0 * i) / hd);
    for (int p = 0; p < ctx_; p++) { const double a = p * inv; cs[(size_t)p * half + i] = (float)std::cos(a); sn[(size_t)p * half + i] = (float)std::sin(a); }
  }
  cos_ = (float *)dalloc(cs.size() * 4); sin_ = (float *)dalloc(sn.size() * 4);
  QPH_CK(hipMemcpy(cos_, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
  QPH_CK(hipMemcpy(sin_, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  QPH_CK(hipHostMalloc((void **)&hctl_, kRing * sizeof(Ctl), hipHostMallocDefault));
  QPH_CK(hipHostMalloc((void **)&hout_, 4ull * std::max(V, d), hipHostMallocDefault));
  QPH_CK(hipHostMalloc((void **)&htok_, 4ull * (ctx_ + 1), hipHostMallocDefault));
  QPH_CK(hipHostMalloc((void **)&htopk_, 8ull * kTopkMax, hipHostMallocDefault));
  {
    const size_t keys = topk_scratch_keys(V, std::min(kTopkMax, V));
    topk_a_ = (uint64_t *)dalloc(8 * keys); topk_b_ = (uint64_t *)dalloc(8 * keys);
    topk_val_ = (float *)dalloc(8ull * kTopkMax); topk_idx_ = (int *)(topk_val_ + kTopkMax);   // one copy back
  }
  QPH_CK(hipHostMalloc((void **)&hstatus_, sizeof(int), hipHostMallocMapped | hipHostMallocCoherent));
  *hstatus_ = 0;
  QPH_CK(hipHostGetDevicePointer((void **)&dstatus_, hstatus_, 0));
  memset(hctl_, 0, kRing * sizeof(Ctl));
  QPH_CK(hipMemset(ctl_, 0, sizeof(Ctl)));
  build_graphs();
}

HipLlama::~HipLlama() {
  if (st_) (void)hipStreamSynchronize(st_);
  for (hipGraphExec_t g : {g_state_, g_logits_, g_greedy_, g_ex_state_, g_ex_logits_, g_ex_greedy_, g_lm_state_,
                           g_lm_logits_, g_lm_greedy_})
    if (g) (void)hipGraphExecDestroy(g);
  for (auto &set : g_fs_)
    for (hipGraphExec_t g : set)
      if (g) (void)hipGraphExecDestroy(g);
  for (void *p : allocs_) (void)hipFree(p);
  if (hctl_) (void)hipHostFree(hctl_);
  if (hout_) (void)hipHostFree(hout_);
  if (htok_) (void)hipHostFree(htok_);
  if (htopk_) (void)hipHostFree(htopk_);
  if (hstatus_) (void)hipHostFree(hstatus_);
  if (st_) (void)hipStreamDestroy(st_);
}

// the decode q / k / v launch's epilogue: RoPE on q and k at ctl->pos, fp16 k / v rows into this layer's caches
void HipLlama::qkv_rope(MvArgs &a, uint16_t *kc, uint16_t *vc) const {
  a.rope[0] = a.rope[1] = 1; a.rope[2] = 0;
  a.cache[0] = nullptr; a.cache[1] = kc; a.cache[2] = vc;
  a.cache_ld = kvd_; a.hd = cfg_.head_dim; a.cos_t = cos_; a.sin_t = sin_; a.ctl = ctl_;
  a.q16[0] = q16_; a.q16[1] = a.q16[2] = nullptr;
}

void HipLlama::enqueue_layer(int l) {
  const Layer &ly = layers_[l];
  const int cap = 1 << 20;
  const float eps = cfg_.rms_eps;
  uint16_t *kc = kc_ + (size_t)l * ctx_ * kvd_, *vc = vc_ + (size_t)l * ctx_ * kvd_;
  {  // RMSNorm + q/k/v (+ bias), RoPE on q / k, fp16 k / v rows into the caches
    MvArgs a{}; a.m[0] = ly.wq; a.m[1] = ly.wk; a.m[2] = ly.wv; a.nseg = 3; a.x = x_; a.norm_w = ly.an; a.eps = eps;
    a.out[0] = q_; a.out[1] = k_; a.out[2] = v_; a.bias[0] = ly.bq; a.bias[1] = ly.bk; a.bias[2] = ly.bv;
    qkv_rope(a, kc, vc);
    a.stamps = gst_take("qkv", kGstWaves, 4, 0, 3); a.stamp_waves = kGstWaves;
    mv_plan(a, EPI_STORE); QPH_CK(launch_matvec(PRO_NORM, EPI_STORE, a, cap, st_));
  }
  AttnArgs at{}; at.q = q_; at.q16 = q16_; at.ctx = ctx_; at.kc = kc; at.vc = vc; at.ctl = ctl_; at.part = part_;
  at.att = att_;
  at.nh = cfg_.heads; at.nkv = cfg_.kv_heads; at.hd = cfg_.head_dim; at.max_chunks = max_chunks_; at.counters = counters_;
  at.single_max = attn_single_; at.split_pos = attn_split_pos_; at.status = dstatus_; at.spin_limit = attn_spin_;
  at.force_late = attn_force_late_; at.merge_sep = lm_ ? lm_splits_ : 0; at.early = fuse_ ? early_ : 0;
  if (fuse_ && awo_rows_) {   // every group's attention and whole wo rows + residual in one launch
    AwoArgs w{}; w.wo = ly.wo; w.x = x_;
    QPH_CK(launch_attn_wo_rows(at, w, st_));
  } else if (fuse_ && awo_sum_) {
    // attention and the wo product per kv group in one launch; each row chunk's last workgroup adds the group parts
    // to the residual stream
    AwoArgs w{}; w.wo = ly.wo; w.part = awo_part_; w.x = x_; w.counters = awo_cnt_;
    w.stamps = gst_take("attn_wo", cfg_.kv_heads * awo_rc_, 5, 0, 4);
    QPH_CK(launch_attn_wo(at, w, st_));
  } else if (fuse_) {
    // RoPE, fp16 KV append, attention and the wo product per kv group in one launch; the group partials are added to
    // the residual stream by the gate / up prologue (x + sum of parts, also stored to xs_), down adds into x_ from xs_
    AwoArgs w{}; w.wo = ly.wo; w.part = awo_part_;
    QPH_CK(launch_attn_wo(at, w, st_));
    MvArgs a{}; a.m[0] = ly.wg; a.m[1] = ly.wu; a.nseg = 2; a.x = x_; a.norm_w = ly.fn; a.eps = eps; a.out[0] = h_;
    a.part = awo_part_; a.nparts = cfg_.kv_heads; a.pstride = (size_t)cfg_.hidden; a.xsum = xs_; a.split_chain = split_chain_;
    mv_plan(a, EPI_SWIGLU); QPH_CK(launch_matvec(PRO_NORM_SUM, EPI_SWIGLU, a, cap, st_));
    MvArgs b{}; b.m[0] = ly.wd; b.nseg = 1; b.x = h_; b.out[0] = x_; b.resid_in = xs_; b.split_chain = split_chain_;
    mv_plan(b, EPI_RESID); QPH_CK(launch_matvec(PRO_QUANT, EPI_RESID, b, cap, st_));
    return;
  } else {
    QPH_CK(launch_attention(at, st_));   // RoPE, fp16 KV append, split-K attention, merge
    MvArgs a{}; a.m[0] = ly.wo; a.nseg = 1; a.x = att_; a.out[0] = x_;   // wo + residual (one chain: k_attn_wo_rows gives the same bits)
    mv_plan(a, EPI_RESID); QPH_CK(launch_matvec(PRO_QUANT, EPI_RESID, a, cap, st_));
  }
  {  // RMSNorm + gate / up + SwiGLU
    MvArgs a{}; a.m[0] = ly.wg; a.m[1] = ly.wu; a.nseg = 2; a.x = x_; a.norm_w = ly.fn; a.eps = eps; a.out[0] = h_;
    a.split_chain = split_chain_;
    a.stamps = gst_take("gate_up", kGstWaves, 4, 0, 3); a.stamp_waves = kGstWaves;
    mv_plan(a, EPI_SWIGLU); QPH_CK(launch_matvec(PRO_NORM, EPI_SWIGLU, a, cap, st_));
  }
  {  // down + residual (the fp32 block chain split over eight lanes per row)
    MvArgs a{}; a.m[0] = ly.wd; a.nseg = 1; a.x = h_; a.out[0] = x_; a.split_chain = split_chain_;
    a.stamps = gst_take("down", kGstWaves, 4, 0, 3); a.stamp_waves = kGstWaves;
    mv_plan(a, EPI_RESID); QPH_CK(launch_matvec(PRO_QUANT, EPI_RESID, a, cap, st_));
  }
}

void HipLlama::enqueue_layers() {
  QPH_CK(launch_embed(embed_, ctl_, x_, st_));
  for (int l = 0; l < cfg_.layers; l++) enqueue_layer(l);
}

void HipLlama::enqueue_head() {
  MvArgs a{}; a.m[0] = head_; a.nseg = 1; a.x = x_; a.norm_w = fnorm_; a.eps = cfg_.rms_eps; a.out[0] = logits_; a.amax = amax_;
  a.stamps = gst_take("head", kGstWaves, 4, 0, 3); a.stamp_waves = kGstWaves;
  mv_plan(a, EPI_ARGMAX);
  QPH_CK(launch_matvec(PRO_NORM, EPI_ARGMAX, a, head_grid_, st_));
}

// one decode step in the current arithmetic order: parts 0 = layers, 1 = + output head (logits), 2 = + greedy pick
// (ctl advances on the device)
// parts 2 (greedy): the step starts from x already embedded (by the previous greedy step's argmax launch, or by
// greedy_run / time_greedy before the first) and ends by embedding its own token for the next one
void HipLlama::enqueue_step(int parts) {
  if (parts < 2) QPH_CK(launch_embed(embed_, ctl_, x_, st_));
  for (int l = 0; l < cfg_.layers; l++) {
    if (order_) ex_enqueue_layer(l);
    else enqueue_layer(l);
  }
  if (parts >= 1) {
    if (order_) ex_enqueue_head();
    else enqueue_head();
  }
  if (parts >= 2) QPH_CK(launch_argmax_finish(amax_, head_grid_, ctl_, out_tok_, st_, &embed_, x_));
}

hipGraphExec_t HipLlama::capture(int parts, bool fused, bool long_merge, int early) {
  hipGraph_t g = nullptr; hipGraphExec_t ge = nullptr;
  fuse_ = fused; lm_ = long_merge; early_ = early;
  gst_off_ = 0; gst_cur_.clear(); gst_capturing_ = gst_ != nullptr;
  QPH_CK(hipStreamBeginCapture(st_, hipStreamCaptureModeThreadLocal));
  try {
    enqueue_step(parts);
    fuse_ = false; lm_ = false; gst_capturing_ = false;
  } catch (...) {
    fuse_ = false; lm_ = false; gst_capturing_ = false;
    (void)hipStreamEndCapture(st_, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  QPH_CK(hipStreamEndCapture(st_, &g));
  QPH_CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  QPH_CK(hipGraphDestroy(g));
  if (gst_) gst_graphs_.emplace_back(ge, gst_cur_);
  return ge;
}

uint64_t *HipLlama::gst_take(const char *name, int n, int stride, int first, int last) {
  if (!gst_capturing_ || gst_off_ + (size_t)n * stride > gst_cap_) return nullptr;
  gst_cur_.push_back({name, gst_off_, n, stride, first, last});
  uint64_t *p = gst_ + gst_off_;
  gst_off_ += (size_t)n * stride;
  return p;
}

void HipLlama::gst_write(const char *path) {
  const std::vector<GStamp> *recs = nullptr;
  for (const auto &g : gst_graphs_) if (g.first == gst_last_) recs = &g.second;
  if (!recs || recs->empty()) return;
  const GStamp &e = recs->back();
  std::vector<uint64_t> h(e.off + (size_t)e.n * e.stride);
  QPH_CK(hipMemcpy(h.data(), gst_, h.size() * 8, hipMemcpyDeviceToHost));
  FILE *f = fopen(path, "w");
  if (!f) return;
  // one line per launch in enqueue order: kernel, earliest start, latest end (100 MHz realtime ticks; units that did
  // not run, with a zero start, are left out)
  for (const GStamp &r : *recs) {
    uint64_t t0 = ~0ull, t1 = 0;
    for (int u = 0; u < r.n; u++) {
      const uint64_t a = h[r.off + (size_t)u * r.stride + r.first], b = h[r.off + (size_t)u * r.stride + r.last];
      if (!a) continue;
      t0 = std::min(t0, a); t1 = std::max(t1, b);
    }
    if (t1) fprintf(f, "%s %llu %llu\n", r.name, (unsigned long long)t0, (unsigned long long)t1);
  }
  fclose(f);
}

void HipLlama::build_graphs() {
  const char *ng = getenv("QPH_NO_GRAPH");
  // Under rocprofv3 (its tool library is announced in ROCP_TOOL_LIBRARIES) the kernels are enqueued directly: the
  // profiler's interception of graph launches crashed the host process (SIGSEGV in the tool, below hipGraphLaunch, at
  // the first replay) while direct launches of the same kernels profile normally.
  const char *prof = getenv("ROCP_TOOL_LIBRARIES");
  if ((ng && atoi(ng) > 0) || (prof && *prof)) { use_graphs_ = false; return; }
  if (getenv("QPH_GRAPH_STAMPS")) {   // measurement hook: one step's launches, each its own region
    gst_cap_ = (size_t)(4 * cfg_.layers + 2) * 4 * kGstWaves;
    gst_ = (uint64_t *)dalloc(gst_cap_ * 8);
    QPH_CK(hipMemset(gst_, 0, gst_cap_ * 8));
  }
  g_state_ = capture(0);
  g_logits_ = capture(1);
  g_greedy_ = capture(2);
  if (awo_max_ > 0)
    for (int e = 1; e <= kEarlyMax; e++) {
      if (32 * (e - 1) >= awo_max_) break;   // no fused context needs this many early blocks
      for (int p = 0; p < 3; p++) g_fs_[e][p] = capture(p, true, false, e);
    }
  if (lm_min_ > 0) {
    g_lm_state_ = capture(0, false, true); g_lm_logits_ = capture(1, false, true); g_lm_greedy_ = capture(2, false, true);
  }
}

// pos: the position this step writes (its context is pos + 1 positions); contexts up to awo_max_ take the fused
// attention + wo kernel
void HipLlama::run_step(int parts, int pos) {
  const bool fused = !order_ && pos + 1 <= awo_max_;
  const bool lm = !order_ && !fused && lm_min_ > 0 && pos + 1 >= lm_min_;
  if (use_graphs_) {
    hipGraphExec_t g = order_ ? (parts == 0 ? g_ex_state_ : parts == 1 ? g_ex_logits_ : g_ex_greedy_)
                       : fused ? g_fs_[early_for(pos)][parts]
                       : lm    ? (parts == 0 ? g_lm_state_ : parts == 1 ? g_lm_logits_ : g_lm_greedy_)
                               : (parts == 0 ? g_state_ : parts == 1 ? g_logits_ : g_greedy_);
    QPH_CK(hipGraphLaunch(g, st_));
    gst_last_ = g;
    return;
  }
  fuse_ = fused; lm_ = lm; early_ = fused ? early_for(pos) : 0;
  enqueue_step(parts);
  fuse_ = false; lm_ = false; early_ = 0;
}

// Called after every wait for the stream, with pos_ already counting every step enqueued so far: a decode attention
// merger whose bounded wait for the other splits' partials ran out wrote NaN outputs and set the status word.  The split
// counters may then be stale, so they are cleared before the error is raised.  The failed step may be any step since the
// last clean check (state-only steps run up to 128 ahead of a wait), and every later step read its cache rows, so the
// position goes back to where that check left it: the cache rows from there on are invalid, the rows before it are not.
void HipLlama::check_status() {
  if (!*(volatile int *)hstatus_) { clean_pos_ = pos_; return; }
  *(volatile int *)hstatus_ = 0;
  pos_ = clean_pos_;
  QPH_CK(hipMemsetAsync(counters_, 0, 8ull * cfg_.kv_heads, st_));
  QPH_CK(hipStreamSynchronize(st_));
  throw std::runtime_error("decode attention: a split merge timed out waiting for its partials; this call's outputs are invalid");
}

void HipLlama::write_ctl(int tok, int pos) {
  // ring of pinned slots: a slot is rewritten only after kRing / 2 later steps, and the host waits for the stream every
  // kRing / 2 steps, so a copy still in flight never sees its source change (the reference's scheme,
  // model_llama_cuda.cu:530-533)
  Ctl &c = hctl_[slot_ % kRing];
  c.tok = tok; c.pos = pos; c.n_out = 0; c.pad = 0;
  QPH_CK(hipMemcpyAsync(ctl_, &c, sizeof(Ctl), hipMemcpyHostToDevice, st_));
  slot_++;
  if (slot_ % (kRing / 2) == 0) { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
}

void HipLlama::step(int tok, int want, float *out) {
  if (pos_ >= ctx_) throw std::runtime_error("context window full (" + std::to_string(ctx_) + " tokens)");
  if (tok < 0 || tok >= cfg_.vocab) throw std::runtime_error("token id out of range");
  write_ctl(tok, pos_);
  if (want == 1 || want == 3) {   // 3 (internal): logits left on the device
    run_step(1, pos_);
    if (want == 1) QPH_CK(hipMemcpyAsync(hout_, logits_, 4ull * cfg_.vocab, hipMemcpyDeviceToHost, st_));
  } else {
    run_step(0, pos_);
    if (want == 2) {
      if (order_) ex_norm(x_, fnorm_, xn_, 1, cfg_.hidden);
      else QPH_CK(launch_rmsnorm(x_, fnorm_, cfg_.hidden, cfg_.rms_eps, xn_, st_));
      QPH_CK(hipMemcpyAsync(hout_, xn_, 4ull * cfg_.hidden, hipMemcpyDeviceToHost, st_));
    }
  }
  pos_++;
  if (want == 1 || want == 2) {
    { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
    if (out) memcpy(out, hout_, 4ull * (want == 1 ? cfg_.vocab : cfg_.hidden));
  }
}

void HipLlama::prefill(const int *toks, int n, int want, float *out) {
  if (n <= 0) return;
  if (pos_ + n > ctx_) throw std::runtime_error("context window full (" + std::to_string(ctx_) + " tokens)");
  for (int i = 0; i < n; i++) if (toks[i] < 0 || toks[i] >= cfg_.vocab) throw std::runtime_error("token id out of range");
  const bool force_steps = getenv("QPH_PREFILL_STEPS") != nullptr;   // test hook: the decode-step path
  // one token (the reference's n == 1 case), or q1 layers in the default order: decode steps
  if (n == 1 || (!pf_ok_ && !order_) || force_steps) {
    for (int i = 0; i < n; i++) step(toks[i], i + 1 == n ? want : 0, i + 1 == n ? out : nullptr);
    if (!want) { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
    return;
  }
  if (order_) ex_prefill(toks, n);
  else prefill_batched(toks, n);
  if (want == 1 || want == 3) {   // 3 (internal): logits left on the device
    if (order_) ex_enqueue_head();
    else enqueue_head();
    if (want == 1) QPH_CK(hipMemcpyAsync(hout_, logits_, 4ull * cfg_.vocab, hipMemcpyDeviceToHost, st_));
  } else if (want == 2) {
    if (order_) ex_norm(x_, fnorm_, xn_, 1, cfg_.hidden);
    else QPH_CK(launch_rmsnorm(x_, fnorm_, cfg_.hidden, cfg_.rms_eps, xn_, st_));
    QPH_CK(hipMemcpyAsync(hout_, xn_, 4ull * cfg_.hidden, hipMemcpyDeviceToHost, st_));
  }
  if (want == 3) return;   // the caller works on the device logits next
  { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
  if (want && out) memcpy(out, hout_, 4ull * (want == 1 ? cfg_.vocab : cfg_.hidden));
}

// The prompt in chunks of up to pf_cap_ tokens, each layer as matrix products (model_llama.cpp:66-130): per chunk the
// embeddings, then per layer RMSNorm + quantise -> q / k / v products (+ bias) -> RoPE and the fp16 cache rows ->
// causal attention -> quantise -> wo product into the residual -> RMSNorm + quantise -> gate product, up product
// with SwiGLU in its store -> quantise -> down product into the residual.  Leaves the last token's hidden state in x_.
void HipLlama::prefill_batched(const int *toks, int n) {
  // QPH_PF_UNFUSED=bits (test hook): 1 q's RoPE, 2 the attention output's quantisation, 4 the SwiGLU output's
  // quantisation as launches of their own, for bit-for-bit comparisons with the fused kernels
  const int unfused = getenv("QPH_PF_UNFUSED") ? atoi(getenv("QPH_PF_UNFUSED")) : 0;
  const int d = cfg_.hidden, ff = cfg_.ffn, nb_ld = pf_ldq_ / 128 + 1;
  const float eps = cfg_.rms_eps;
  auto quant = [&](int pro, const float *x, int ldx, const float *w, int cols, int B) {
    PfQuantArgs a{}; a.x = x; a.ldx = ldx; a.norm_w = w; a.eps = eps; a.cols = cols;
    a.xh = pf_xh_; a.xl = pf_xl_; a.ldq = pf_ldq_; a.xb = pf_xb_; a.ldb = nb_ld; a.xg = pf_xg_; a.ldg = pf_ldg_;
    a.xbt = pf_xbt_; a.ldbt = pf_ldbt_;
    QPH_CK(launch_pf_quant(pro, a, B, st_));
  };
  auto gemm = [&](const DMat &m, float *y, int ldy, const float *bias, bool resid, int B, const float *gate = nullptr) {
    GemmArgs a{}; a.kind = m.kind; a.w = (const int8_t *)m.q; a.scale = (const float *)m.s; a.rows = m.rows; a.cols = m.cols;
    a.wsum = m.rs; a.xbt = pf_xbt_; a.ldbt = pf_ldbt_; a.q4ns = m.q4ns; a.q4sc = m.q4sc; a.xg = pf_xg_; a.ldg = pf_ldg_;
    a.xh = pf_xh_; a.xl = pf_xl_; a.xb = pf_xb_; a.ntok = B; a.ldq = pf_ldq_; a.ldb = nb_ld;
    a.y = y; a.ldy = ldy; a.bias = bias; a.resid = resid ? 1 : 0; a.gate = gate;
    QPH_CK(launch_gemm(a, st_));
  };
  // q / k / v: runs of consecutive matrices of one kind share a launch (q8 files: one launch; q4m: q + k, then v)
  auto gemm_qkv = [&](const Layer &ly, int B) {
    const DMat *m[3] = {&ly.wq, &ly.wk, &ly.wv};
    float *y[3] = {pf_q_, pf_k_, pf_v_};
    const int ld[3] = {qd_, kvd_, kvd_};
    const float *bias[3] = {ly.bq, ly.bk, ly.bv};
    for (int i = 0; i < 3;) {
      int j = i + 1;
      while (j < 3 && m[j]->kind == m[i]->kind && m[j]->cols == m[i]->cols) j++;
      if (j - i == 1 || (m[i]->kind != MK_Q8 && m[i]->kind != MK_Q4)) { gemm(*m[i], y[i], ld[i], bias[i], false, B); i++; continue; }
      GemmArgs a{}; a.kind = m[i]->kind; a.cols = m[i]->cols; a.xbt = pf_xbt_; a.ldbt = pf_ldbt_; a.xg = pf_xg_; a.ldg = pf_ldg_;
      a.xh = pf_xh_; a.xl = pf_xl_; a.xb = pf_xb_; a.ntok = B; a.ldq = pf_ldq_; a.ldb = nb_ld;
      a.nseg = j - i;
      for (int s = i; s < j; s++)
        a.seg[s - i] = GemmSeg{(const int8_t *)m[s]->q, (const float *)m[s]->s, m[s]->rs, m[s]->q4ns, m[s]->q4sc, bias[s], y[s], m[s]->rows, ld[s]};
      QPH_CK(launch_gemm(a, st_));
      i = j;
    }
  };
  int B = 0;
  for (int s0 = 0; s0 < n; s0 += B) {
    B = std::min(pf_cap_, n - s0);
    const int p0 = pos_;
    QPH_CK(hipMemcpyAsync(pf_tok_, toks + s0, 4ull * B, hipMemcpyHostToDevice, st_));
    QPH_CK(launch_pf_embed(embed_, pf_tok_, B, pf_x_, d, st_));
    for (int l = 0; l < cfg_.layers; l++) {
      const Layer &ly = layers_[l];
      uint16_t *kc = kc_ + (size_t)l * ctx_ * kvd_, *vc = vc_ + (size_t)l * ctx_ * kvd_;
      quant(PRO_NORM, pf_x_, d, ly.an, d, B);
      gemm_qkv(ly, B);
      // q's RoPE happens in the attention kernel; at head dim 128 (one head = one quantisation block) that kernel also
      // quantises its output for a q8 wo
      PfRopeArgs r{}; r.q = pf_q_; r.ldq = qd_; r.k = pf_k_; r.v = pf_v_; r.ldk = kvd_; r.cos_t = cos_; r.sin_t = sin_;
      r.kc = kc; r.vc = vc; r.p0 = p0; r.nh = cfg_.heads; r.nkv = cfg_.kv_heads; r.hd = cfg_.head_dim; r.skip_q = !(unfused & 1);
      QPH_CK(launch_pf_rope(r, B, st_));
      PfAttnArgs t{}; t.q = pf_q_; t.ldq = qd_; t.kc = kc; t.vc = vc; t.att = pf_att_; t.lda = qd_;
      t.ntok = B; t.p0 = p0; t.nh = cfg_.heads; t.nkv = cfg_.kv_heads; t.hd = cfg_.head_dim;
      if (!(unfused & 1)) { t.cos_t = cos_; t.sin_t = sin_; }
      const bool att_q = !(unfused & 2) && cfg_.head_dim == 128 && ly.wo.kind == MK_Q8;
      if (att_q) {
        t.oh = pf_xh_; t.ol = pf_xl_; t.ob = pf_xb_; t.obt = pf_xbt_; t.ldo = pf_ldq_; t.ldb = nb_ld; t.ldbt = pf_ldbt_;
      }
      QPH_CK(launch_pf_attn(t, st_));
      if (!att_q) quant(PRO_QUANT, pf_att_, qd_, nullptr, qd_, B);
      gemm(ly.wo, pf_x_, d, nullptr, true, B);
      quant(PRO_NORM, pf_x_, d, ly.fn, d, B);
      bool fused = false;   // h = silu(gate) * up quantised by the product's store, straight into the second planes
      if (ly.wg.kind == MK_Q8 && ly.wu.kind == MK_Q8) {   // gate and up in one launch, only h = silu(gate) * up stored
        GemmArgs a{}; a.kind = MK_Q8; a.w = (const int8_t *)ly.wg.q; a.scale = (const float *)ly.wg.s; a.wsum = ly.wg.rs;
        a.w2 = (const int8_t *)ly.wu.q; a.scale2 = (const float *)ly.wu.s; a.wsum2 = ly.wu.rs;
        a.rows = ff; a.cols = d; a.xbt = pf_xbt_; a.ldbt = pf_ldbt_; a.xh = pf_xh_; a.xl = pf_xl_; a.xb = pf_xb_; a.ntok = B;
        a.ldq = pf_ldq_; a.ldb = nb_ld; a.y = pf_g_; a.ldy = ff;
        fused = !(unfused & 4) && ly.wd.kind == MK_Q8 && ff % 128 == 0 && gemm_uses_32x32(a);
        if (fused) { a.oh = pf_xh2_; a.ol = pf_xl2_; a.ob = pf_xb2_; a.obt = pf_xbt2_; }
        QPH_CK(launch_gemm(a, st_));
      } else {
        gemm(ly.wg, pf_g_, ff, nullptr, false, B);
        gemm(ly.wu, pf_g_, ff, nullptr, false, B, pf_g_);   // h = silu(gate) * up, in place over the gate product
      }
      if (fused) {
        GemmArgs a{}; a.kind = MK_Q8; a.w = (const int8_t *)ly.wd.q; a.scale = (const float *)ly.wd.s; a.rows = ly.wd.rows;
        a.cols = ly.wd.cols; a.wsum = ly.wd.rs; a.xbt = pf_xbt2_; a.ldbt = pf_ldbt_; a.xh = pf_xh2_; a.xl = pf_xl2_;
        a.xb = pf_xb2_; a.ntok = B; a.ldq = pf_ldq_; a.ldb = nb_ld; a.y = pf_x_; a.ldy = d; a.resid = 1;
        QPH_CK(launch_gemm(a, st_));
      } else {
        quant(PRO_QUANT, pf_g_, ff, nullptr, ff, B);
        gemm(ly.wd, pf_x_, d, nullptr, true, B);
      }
    }
    pos_ += B;
  }
  QPH_CK(hipMemcpyAsync(x_, pf_x_ + (size_t)(B - 1) * d, 4ull * d, hipMemcpyDeviceToDevice, st_));
}

void HipLlama::topk_to_host(int M, int *idx, float *val) {
  QPH_CK(launch_topk(logits_, cfg_.vocab, M, topk_a_, topk_b_, topk_idx_, topk_val_, st_));
  // values at [0, M), indices at [kTopkMax, kTopkMax + M) of one device buffer: one copy of the used span
  QPH_CK(hipMemcpyAsync(htopk_, topk_val_, 4ull * (kTopkMax + M), hipMemcpyDeviceToHost, st_));
  { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
  memcpy(val, htopk_, 4ull * M);
  memcpy(idx, htopk_ + kTopkMax, 4ull * M);
}
void HipLlama::step_topk(int tok, int M, int *idx, float *val) {
  if (M < 1 || M > std::min(kTopkMax, cfg_.vocab)) throw std::runtime_error("top-M: M must be in [1, min(512, vocab)]");
  step(tok, 3, nullptr);
  topk_to_host(M, idx, val);
}
void HipLlama::prefill_topk(const int *toks, int n, int M, int *idx, float *val) {
  if (M < 1 || M > std::min(kTopkMax, cfg_.vocab)) throw std::runtime_error("top-M: M must be in [1, min(512, vocab)]");
  if (n <= 0) throw std::runtime_error("prefill: no tokens");
  prefill(toks, n, 3, nullptr);
  topk_to_host(M, idx, val);
}

int HipLlama::greedy_run(int tok, int n, int *out) {
  n = std::min(n, ctx_ - pos_);
  if (n <= 0) return 0;
  if (tok < 0 || tok >= cfg_.vocab) throw std::runtime_error("token id out of range");
  write_ctl(tok, pos_);
  QPH_CK(launch_embed(embed_, ctl_, x_, st_));   // the first step's input; each step embeds the next one's
  for (int i = 0; i < n; i++) run_step(2, pos_ + i);
  QPH_CK(hipMemcpyAsync(htok_, out_tok_, 4ull * n, hipMemcpyDeviceToHost, st_));
  pos_ += n;
  { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
  memcpy(out, htok_, 4ull * n);
  return n;
}

void HipLlama::prefill_all(const int *toks, int n, float *logits) {
  if (pos_ + n > ctx_) throw std::runtime_error("context window full (" + std::to_string(ctx_) + " tokens)");
  for (int i = 0; i < n; i++) step(toks[i], 1, logits + (size_t)i * cfg_.vocab);
}

void HipLlama::set_pos(int pos) {
  if (pos < 0 || pos > ctx_) throw std::runtime_error("position out of range");
  pos_ = pos; clean_pos_ = std::min(clean_pos_, pos);
}

void HipLlama::snapshot(uint8_t *buf, int64_t cap) {
  if (cap < snapshot_size()) throw std::runtime_error("snapshot buffer too small");
  { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
  memcpy(buf, &pos_, 4); uint8_t *p = buf + 4; const size_t nb = (size_t)pos_ * kvd_ * 2;
  for (int l = 0; l < cfg_.layers; l++)
    for (uint16_t *c : {kc_, vc_}) { QPH_CK(hipMemcpy(p, c + (size_t)l * ctx_ * kvd_, nb, hipMemcpyDeviceToHost)); p += nb; }
}

void HipLlama::restore(const uint8_t *buf, int64_t n) {
  if (n < 4) throw std::runtime_error("snapshot too short");
  int pos; memcpy(&pos, buf, 4);
  if (pos < 0 || pos > ctx_) throw std::runtime_error("snapshot position out of range");
  const size_t nb = (size_t)pos * kvd_ * 2;
  if (n < (int64_t)(4 + 2 * nb * cfg_.layers)) throw std::runtime_error("snapshot too short");
  { QPH_CK(hipStreamSynchronize(st_)); check_status(); }
  const uint8_t *p = buf + 4;
  for (int l = 0; l < cfg_.layers; l++)
    for (uint16_t *c : {kc_, vc_}) { QPH_CK(hipMemcpy(c + (size_t)l * ctx_ * kvd_, p, nb, hipMemcpyHostToDevice)); p += nb; }
  pos_ = pos; clean_pos_ = pos;
}

// ------------------------------------------------------------------ reference-order mode
// The reference CPU path's arithmetic order everywhere (exact.hip holds what the default kernels do differently):
// RMSNorm's sequential sum, attention over 64-position chunks with an ordered merge (decode) or full rows (prompt),
// rows_q4 for the q4 products, the prompt's products in mm_q8 / mm_q4 order for the first B - B % 4 vectors of each
// 64-token batch, and the C library's expf on softmax tails.  q8 decode products, quantisation, RoPE, the fp16 cache
// rows and every epilogue are the default kernels, which already follow the reference's order.
void HipLlama::set_order(int mode) {
  if (mode != 0 && mode != 1) throw std::runtime_error("order: mode must be 0 (default) or 1 (reference order)");
  if (mode == 1) {
    if (head_.kind != MK_Q8 && head_.kind != MK_Q4) throw std::runtime_error("order: reference order needs a q8 or q4 output head");
    if (!ex_part_) {
      ex_ncmax_ = (ctx_ + 63) / 64;
      ex_part_ = (float *)dalloc(4ull * cfg_.heads * ex_ncmax_ * (cfg_.head_dim + 2));
      ex_qr_ = (float *)dalloc(4ull * qd_);
      const int B = std::min(64, pf_cap_);
      ex_u_ = (float *)dalloc(4ull * B * cfg_.ffn);
      ex_xn_ = (float *)dalloc(4ull * B * cfg_.hidden);
    }
  }
  QPH_CK(hipStreamSynchronize(st_));
  order_ = mode;
  if (mode == 1 && use_graphs_ && !g_ex_state_) {
    g_ex_state_ = capture(0);
    g_ex_logits_ = capture(1);
    g_ex_greedy_ = capture(2);
  }
}

void HipLlama::ex_norm(const float *x, const float *w, float *out, int rows, int ldx) {
  QPH_CK(launch_ex_rmsnorm(x, ldx, w, cfg_.hidden, cfg_.rms_eps, out, cfg_.hidden, rows, st_));
}

// y [ntok][ldy] = m x_t (+ bias, or += when resid) in the reference's order; x [ntok][ldx] is quantised into the prompt
// planes first unless `quantised` says they already hold it
void HipLlama::ex_product(const DMat &m, const float *x, int ldx, int ntok, int mm_below, float *y, int ldy,
                          const float *bias, bool resid, bool quantised) {
  const int nb_ld = pf_ldq_ / 128 + 1;
  if (!quantised) {
    PfQuantArgs q{}; q.x = x; q.ldx = ldx; q.cols = m.cols; q.xh = pf_xh_; q.xl = pf_xl_; q.ldq = pf_ldq_;
    q.xb = pf_xb_; q.ldb = nb_ld;
    QPH_CK(launch_pf_quant(PRO_QUANT, q, ntok, st_));
  }
  ExGemmArgs a{}; a.kind = m.kind; a.w = m.q; a.scale = (const float *)m.s; a.s16 = (const uint16_t *)m.s;
  a.rows = m.rows; a.cols = m.cols; a.xh = pf_xh_; a.xl = pf_xl_; a.ldq = pf_ldq_; a.xb = pf_xb_; a.ldb = nb_ld;
  a.ntok = ntok; a.mm_below = mm_below; a.tt = ntok == 1 ? 1 : 16; a.y = y; a.ldy = ldy; a.bias = bias; a.resid = resid ? 1 : 0;
  QPH_CK(launch_ex_gemm(a, st_));
}

void HipLlama::ex_enqueue_layer(int l) {
  const Layer &ly = layers_[l];
  const int d = cfg_.hidden, ff = cfg_.ffn, cap = 1 << 20;
  uint16_t *kc = kc_ + (size_t)l * ctx_ * kvd_, *vc = vc_ + (size_t)l * ctx_ * kvd_;
  // the q8 matrices of a group share one launch of the default matvec (PRO_QUANT: x is already normalised); q4 ones
  // take the rows_q4-order product
  auto group = [&](const DMat *const *m, float *const *y, const float *const *bias, int n, const float *x, int ldx) {
    MvArgs a{}; a.x = x;
    bool quantised = false;
    for (int s = 0; s < n; s++)
      if (m[s]->kind == MK_Q8) { a.m[a.nseg] = *m[s]; a.out[a.nseg] = y[s]; a.bias[a.nseg] = bias[s]; a.nseg++; }
    if (a.nseg) { mv_plan(a, EPI_STORE); QPH_CK(launch_matvec(PRO_QUANT, EPI_STORE, a, cap, st_)); }
    for (int s = 0; s < n; s++)
      if (m[s]->kind != MK_Q8) { ex_product(*m[s], x, ldx, 1, 0, y[s], 0, bias[s], false, quantised); quantised = true; }
  };
  auto resid = [&](const DMat &m, const float *x, int cols) {
    if (m.kind == MK_Q8) {
      MvArgs a{}; a.m[0] = m; a.nseg = 1; a.x = x; a.out[0] = x_;
      mv_plan(a, EPI_RESID); QPH_CK(launch_matvec(PRO_QUANT, EPI_RESID, a, cap, st_));
    } else ex_product(m, x, cols, 1, 0, x_, 0, nullptr, true, false);
  };
  ex_norm(x_, ly.an, xn_, 1, d);
  {
    const DMat *m[3] = {&ly.wq, &ly.wk, &ly.wv};
    float *y[3] = {q_, k_, v_};
    const float *b[3] = {ly.bq, ly.bk, ly.bv};
    group(m, y, b, 3, xn_, d);
  }
  ExRopeArgs r{}; r.q = q_; r.k = k_; r.v = v_; r.qr = ex_qr_; r.cos_t = cos_; r.sin_t = sin_; r.ctl = ctl_;
  r.kc = kc; r.vc = vc; r.nh = cfg_.heads; r.nkv = cfg_.kv_heads; r.hd = cfg_.head_dim;
  QPH_CK(launch_ex_rope(r, st_));
  ExAttnArgs t{}; t.qr = ex_qr_; t.kc = kc; t.vc = vc; t.ctl = ctl_; t.part = ex_part_; t.att = att_;
  t.nh = cfg_.heads; t.nkv = cfg_.kv_heads; t.hd = cfg_.head_dim; t.ncmax = ex_ncmax_;
  QPH_CK(launch_ex_attention(t, st_));
  resid(ly.wo, att_, qd_);
  ex_norm(x_, ly.fn, xn_, 1, d);
  {
    const DMat *m[2] = {&ly.wg, &ly.wu};
    float *y[2] = {h_, ex_u_};
    const float *b[2] = {nullptr, nullptr};
    group(m, y, b, 2, xn_, d);
  }
  QPH_CK(launch_ex_silu(h_, ex_u_, ff, ff, 1, st_));
  resid(ly.wd, h_, ff);
}

void HipLlama::ex_enqueue_head() {
  ex_norm(x_, fnorm_, xn_, 1, cfg_.hidden);
  if (head_.kind == MK_Q8) {   // rows_q8 (the argmax matvec's order) with the greedy pick's partials
    MvArgs a{}; a.m[0] = head_; a.nseg = 1; a.x = xn_; a.out[0] = logits_; a.amax = amax_;
    mv_plan(a, EPI_ARGMAX);
    QPH_CK(launch_matvec(PRO_QUANT, EPI_ARGMAX, a, head_grid_, st_));
  } else {   // a q4 head (--q4-head files): rows_q4's order, then the partials from the logits
    ex_product(head_, xn_, cfg_.hidden, 1, 0, logits_, 0, nullptr, false, false);
    QPH_CK(launch_ex_argmax_parts(logits_, cfg_.vocab, amax_, head_grid_, st_));
  }
}

// the prompt in the reference's batches of 64 tokens (model_llama.cpp:66-130)
void HipLlama::ex_prefill(const int *toks, int n) {
  const int d = cfg_.hidden, ff = cfg_.ffn, PB = std::min(64, pf_cap_);
  int B = 0;
  for (int s0 = 0; s0 < n; s0 += B) {
    B = std::min(PB, n - s0);
    const int p0 = pos_, b4 = B - B % 4;
    QPH_CK(hipMemcpyAsync(pf_tok_, toks + s0, 4ull * B, hipMemcpyHostToDevice, st_));
    QPH_CK(launch_pf_embed(embed_, pf_tok_, B, pf_x_, d, st_));
    for (int l = 0; l < cfg_.layers; l++) {
      const Layer &ly = layers_[l];
      uint16_t *kc = kc_ + (size_t)l * ctx_ * kvd_, *vc = vc_ + (size_t)l * ctx_ * kvd_;
      ex_norm(pf_x_, ly.an, ex_xn_, B, d);
      ex_product(ly.wq, ex_xn_, d, B, b4, pf_q_, qd_, ly.bq, false, false);
      ex_product(ly.wk, ex_xn_, d, B, b4, pf_k_, kvd_, ly.bk, false, true);
      ex_product(ly.wv, ex_xn_, d, B, b4, pf_v_, kvd_, ly.bv, false, true);
      PfRopeArgs r{}; r.q = pf_q_; r.ldq = qd_; r.k = pf_k_; r.v = pf_v_; r.ldk = kvd_; r.cos_t = cos_; r.sin_t = sin_;
      r.kc = kc; r.vc = vc; r.p0 = p0; r.nh = cfg_.heads; r.nkv = cfg_.kv_heads; r.hd = cfg_.head_dim;
      QPH_CK(launch_pf_rope(r, B, st_));
      ExPfAttnArgs t{}; t.q = pf_q_; t.ldq = qd_; t.kc = kc; t.vc = vc; t.att = pf_att_; t.lda = qd_;
      t.p0 = p0; t.nh = cfg_.heads; t.nkv = cfg_.kv_heads; t.hd = cfg_.head_dim;
      QPH_CK(launch_ex_pf_attn(t, B, st_));
      ex_product(ly.wo, pf_att_, qd_, B, b4, pf_x_, d, nullptr, true, false);
      ex_norm(pf_x_, ly.fn, ex_xn_, B, d);
      ex_product(ly.wg, ex_xn_, d, B, b4, pf_g_, ff, nullptr, false, false);
      ex_product(ly.wu, ex_xn_, d, B, b4, ex_u_, ff, nullptr, false, true);
      QPH_CK(launch_ex_silu(pf_g_, ex_u_, ff, ff, B, st_));
      ex_product(ly.wd, pf_g_, ff, B, b4, pf_x_, d, nullptr, true, false);
    }
    pos_ += B;
  }
  QPH_CK(hipMemcpyAsync(x_, pf_x_ + (size_t)(B - 1) * d, 4ull * d, hipMemcpyDeviceToDevice, st_));
}

float HipLlama::time_greedy(int tok, int n) {
  n = std::min(n, ctx_ - pos_);
  if (n <= 0) throw std::runtime_error("context window full");
  hipEvent_t e0, e1;
  QPH_CK(hipEventCreate(&e0)); QPH_CK(hipEventCreate(&e1));
  write_ctl(tok, pos_);
  QPH_CK(hipEventRecord(e0, st_));
  QPH_CK(launch_embed(embed_, ctl_, x_, st_));   // the first step's input; each step embeds the next one's
  for (int i = 0; i < n; i++) run_step(2, pos_ + i);
  QPH_CK(hipEventRecord(e1, st_));
  pos_ += n;
  QPH_CK(hipEventSynchronize(e1)); check_status();
  float ms = 0; QPH_CK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0); (void)hipEventDestroy(e1);
  if (const char *gp = getenv("QPH_GRAPH_STAMPS")) if (gst_) gst_write(gp);
  return ms;
}

static double mat_bytes(const DMat &m) {
  if (m.kind == MK_Q8) return (double)m.rows * m.cols + 4.0 * m.rows;
  if (m.kind == MK_Q1) return (double)m.rows * m.cols / 8 + 2.0 * m.rows * (m.cols / 128);
  return (double)m.rows * m.cols / 2 + 2.0 * m.rows * (m.cols / 32);
}

float HipLlama::time_kernel(int which, int iters, double *bytes) {
  if (iters <= 0) iters = 1;
  // consecutive launches walk the layers, as the token loop does, so no launch finds its weights in the
  // 256 MiB last-level cache from the previous one
  // QPH_TK_LAYERS (measurement hook): walk only that many layers, so repeated launches find their weights cached
  const char *tkl = getenv("QPH_TK_LAYERS");
  const int L = tkl ? std::max(1, std::min(cfg_.layers, atoi(tkl))) : cfg_.layers, d = cfg_.hidden, cap = 1 << 20;
  int li = 0;
  const float eps = cfg_.rms_eps;
  write_ctl(0, std::min(pos_, ctx_ - 1));
  // QPH_AWO_STAMPS=file (measurement hook): the fused attention + wo kernel's per-workgroup realtime stamps of the
  // last timed launch, written to that file as text
  const char *stf = which == 6 ? getenv("QPH_AWO_STAMPS") : which == 5 ? getenv("QPH_ATTN_STAMPS") : nullptr;
  uint64_t *stamps = stf ? (uint64_t *)dalloc(5 * 8 * 4096) : nullptr;
  if (stamps) QPH_CK(hipMemset(stamps, 0, 5 * 8 * 4096));
  const char *dme = getenv("QPH_MV_DBG");
  const int dmode = dme ? atoi(dme) : 0;
  // QPH_MV_STAMPS=file (measurement hook): the matvec's per-wave realtime stamps of the last timed launch, as text
  const char *mvs = which <= 4 || which == 7 ? getenv("QPH_MV_STAMPS") : nullptr;
  uint64_t *mv_stamps = mvs ? (uint64_t *)dalloc(4 * 8 * 65536) : nullptr;
  if (mv_stamps) QPH_CK(hipMemset(mv_stamps, 0, 4 * 8 * 65536));
  auto launch = [&]() {
    const Layer &ly = layers_[li];
    li = li + 1 == L ? 0 : li + 1;
    MvArgs a{};
    a.dbg_mode = dmode;
    a.stamps = mv_stamps;
    switch (which) {
      case 0:
        a.m[0] = ly.wg; a.m[1] = ly.wu; a.nseg = 2; a.x = x_; a.norm_w = ly.fn; a.eps = eps; a.out[0] = h_;
        a.split_chain = split_chain_;
        mv_plan(a, EPI_SWIGLU); QPH_CK(launch_matvec(PRO_NORM, EPI_SWIGLU, a, cap, st_)); break;
      case 1:   // as the token loop runs it: into a residual (scratch here), the block chain split
        a.m[0] = ly.wd; a.nseg = 1; a.x = h_; a.out[0] = xn_; a.split_chain = split_chain_;
        mv_plan(a, EPI_RESID); QPH_CK(launch_matvec(PRO_QUANT, EPI_RESID, a, cap, st_)); break;
      case 2:
        a.m[0] = ly.wq; a.m[1] = ly.wk; a.m[2] = ly.wv; a.nseg = 3; a.x = x_; a.norm_w = ly.an; a.eps = eps;
        a.out[0] = q_; a.out[1] = k_; a.out[2] = v_; a.bias[0] = ly.bq; a.bias[1] = ly.bk; a.bias[2] = ly.bv;
        qkv_rope(a, kc_, vc_);
        mv_plan(a, EPI_STORE); QPH_CK(launch_matvec(PRO_NORM, EPI_STORE, a, cap, st_)); break;
      case 3:
        a.m[0] = ly.wo; a.nseg = 1; a.x = att_; a.out[0] = xn_;
        mv_plan(a, EPI_STORE); QPH_CK(launch_matvec(PRO_QUANT, EPI_STORE, a, cap, st_)); break;
      case 4: enqueue_head(); break;
      case 6: {   // fused attention + wo (QPH_AWO_EARLY: the early-load count, else the position's)
        AttnArgs t{}; t.q = q_; t.q16 = q16_; t.ctx = ctx_; t.kc = kc_; t.vc = vc_; t.ctl = ctl_;
        t.early = getenv("QPH_AWO_EARLY") ? atoi(getenv("QPH_AWO_EARLY")) : early_for(std::min(pos_, ctx_ - 1));
        t.part = part_; t.att = att_; t.nh = cfg_.heads; t.nkv = cfg_.kv_heads; t.hd = cfg_.head_dim;
        AwoArgs w{}; w.wo = ly.wo; w.part = awo_part_; w.x = xn_;
        if (awo_rows_) { QPH_CK(launch_attn_wo_rows(t, w, st_)); break; }
        if (!awo_part_) throw std::runtime_error("time_kernel: the fused attention + wo kernel does not take this model");
        w.stamps = stamps;
        if (awo_sum_) w.counters = awo_cnt_;   // adds into xn_ (scratch)
        QPH_CK(launch_attn_wo(t, w, st_)); break;
      }
      case 7:   // gate / up after the fused attention + wo: x + the group parts
        if (!awo_part_) throw std::runtime_error("time_kernel: the fused attention + wo kernel does not take this model");
        a.m[0] = ly.wg; a.m[1] = ly.wu; a.nseg = 2; a.x = x_; a.norm_w = ly.fn; a.eps = eps; a.out[0] = h_;
        a.part = awo_part_; a.nparts = cfg_.kv_heads; a.pstride = (size_t)d; a.xsum = xs_;
        mv_plan(a, EPI_SWIGLU); QPH_CK(launch_matvec(PRO_NORM_SUM, EPI_SWIGLU, a, cap, st_)); break;
      case 5: {
        AttnArgs t{}; t.q = q_; t.q16 = q16_; t.ctx = ctx_; t.kc = kc_; t.vc = vc_; t.ctl = ctl_;
        t.part = part_; t.att = att_; t.nh = cfg_.heads; t.nkv = cfg_.kv_heads; t.hd = cfg_.head_dim;
        t.max_chunks = max_chunks_; t.counters = counters_; t.single_max = attn_single_; t.split_pos = attn_split_pos_;
        t.status = dstatus_; t.spin_limit = attn_spin_; t.stamps = stamps; t.merge_sep = lm_min_ > 0 && pos_ + 1 >= lm_min_ ? lm_splits_ : 0;
        QPH_CK(launch_attention(t, st_)); break;
      }
      default: throw std::runtime_error("time_kernel: unknown kernel id");
    }
  };
  // algorithmic bytes per launch, averaged over the layers (q4 mixes differ by layer)
  double sum = 0;
  for (const Layer &ly : layers_) {
    switch (which) {
      case 0: sum += mat_bytes(ly.wg) + mat_bytes(ly.wu) + 4.0 * d; break;
      case 1: sum += mat_bytes(ly.wd); break;
      case 2: sum += mat_bytes(ly.wq) + mat_bytes(ly.wk) + mat_bytes(ly.wv) + 4.0 * d; break;
      case 3: sum += mat_bytes(ly.wo); break;
      case 4: sum += mat_bytes(head_) + 4.0 * d + 4.0 * cfg_.vocab; break;
      case 5: sum += 4.0 * (double)(pos_ + 1) * kvd_; break;
      case 6: sum += 4.0 * (double)(pos_ + 1) * kvd_ + mat_bytes(ly.wo); break;
      case 7: sum += mat_bytes(ly.wg) + mat_bytes(ly.wu) + 4.0 * d * (1 + cfg_.kv_heads); break;
      default: throw std::runtime_error("time_kernel: unknown kernel id");
    }
  }
  *bytes = sum / L;
  launch();   // warm-up
  hipEvent_t e0, e1;
  QPH_CK(hipEventCreate(&e0)); QPH_CK(hipEventCreate(&e1));
  QPH_CK(hipEventRecord(e0, st_));
  for (int i = 0; i < iters; i++) launch();
  QPH_CK(hipEventRecord(e1, st_));
  QPH_CK(hipEventSynchronize(e1)); check_status();
  float ms = 0; QPH_CK(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0); (void)hipEventDestroy(e1);
  if (mv_stamps) {
    std::vector<uint64_t> h(4 * 65536);
    QPH_CK(hipMemcpy(h.data(), mv_stamps, h.size() * 8, hipMemcpyDeviceToHost));
    if (FILE *f = fopen(mvs, "w")) {
      for (int i = 0; i < 65536 && h[4 * i]; i++)
        fprintf(f, "%llu %llu %llu %llu\n", (unsigned long long)h[4 * i], (unsigned long long)h[4 * i + 1],
                (unsigned long long)h[4 * i + 2], (unsigned long long)h[4 * i + 3]);
      fclose(f);
    }
  }
  if (stamps) {
    std::vector<uint64_t> h(5 * 4096);
    QPH_CK(hipMemcpy(h.data(), stamps, h.size() * 8, hipMemcpyDeviceToHost));
    if (FILE *f = fopen(stf, "w")) {
      if (which == 6)   // start, the wo tile issued (block loops done), attention out, block sums, end
        for (int i = 0; i < cfg_.kv_heads * awo_rc_; i++)
          fprintf(f, "%llu %llu %llu %llu %llu\n", (unsigned long long)h[5 * i], (unsigned long long)h[5 * i + 1],
                  (unsigned long long)h[5 * i + 2], (unsigned long long)h[5 * i + 3], (unsigned long long)h[5 * i + 4]);
      else
        for (int i = 0; i < cfg_.kv_heads * max_chunks_ && 5 * i + 4 < (int)h.size(); i++)
          if (h[5 * i])
            fprintf(f, "%llu %llu %llu %llu %llu\n", (unsigned long long)h[5 * i], (unsigned long long)h[5 * i + 1],
                    (unsigned long long)h[5 * i + 2], (unsigned long long)h[5 * i + 3], (unsigned long long)h[5 * i + 4]);
      fclose(f);
    }
  }
  return ms / iters;
}

}  // namespace qph
