// The HIP Llama model: the host side of the gfx950 token loop, shaped like qp::Model
// (/root/reference/include/qpack/qpack.h:128-171) and the reference GPU model LlamaCuda
// (/root/reference/src/model_llama_cuda.cu:445-632).
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>
#include <vector>

#include "../../../include/qpack_hip.h"
#include "common.hpp"
#include "launch.hpp"

namespace qph {

class HipLlama {
 public:
  HipLlama(const qph_config &cfg, const qph_tensor *tensors, int n, int max_ctx);
  ~HipLlama();
  HipLlama(const HipLlama &) = delete;
  HipLlama &operator=(const HipLlama &) = delete;

  const qph_config &config() const { return cfg_; }
  const RansTiming &load_timing() const { return rans_tm_; }
  int max_ctx() const { return ctx_; }
  int pos() const { return pos_; }

  void step(int tok, int want, float *out);
  void prefill(const int *toks, int n, int want, float *out);
  int greedy_run(int tok, int n, int *out);
  void prefill_all(const int *toks, int n, float *logits);
  // step / prefill whose logits stay on the device and come back as their M largest (index, value) pairs, in the
  // sampler's order (1 <= M <= min(kTopkMax, vocab))
  void step_topk(int tok, int M, int *idx, float *val);
  void prefill_topk(const int *toks, int n, int M, int *idx, float *val);
  void reset() { pos_ = 0; clean_pos_ = 0; }
  bool rewind(int pos) {
    if (pos < 0 || pos > pos_) return false;
    pos_ = pos; clean_pos_ = std::min(clean_pos_, pos); return true;
  }
  void set_pos(int pos);
  int64_t snapshot_size() const { return 4 + 4ll * cfg_.layers * pos_ * kvd_; }
  void snapshot(uint8_t *buf, int64_t cap);
  void restore(const uint8_t *buf, int64_t n);

  // arithmetic order: 0 = this library's kernels (default), 1 = the reference CPU path's order everywhere, so logits,
  // caches and greedy streams are bit-identical to qp::Llama's (slower: a test and verification mode)
  void set_order(int mode);
  int order() const { return order_; }

  float time_greedy(int tok, int n);
  float time_kernel(int which, int iters, double *bytes);

 private:
  struct Layer {
    DMat wq, wk, wv, wo, wg, wu, wd;
    const float *an = nullptr, *fn = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
  };
  qph_config cfg_;
  int ctx_ = 0, kvd_ = 0, qd_ = 0, max_chunks_ = 1, cus_ = 256, head_grid_ = 0;
  int *counters_ = nullptr;
  int attn_single_ = 0, attn_split_pos_ = 0, attn_spin_ = 0;   // attention split policy (0: the kernel's defaults)
  int split_chain_ = 1;   // EPI_RESID matvecs chain their fp32 block sums over 8 lanes per row (QPH_MV_SPLIT=0: one chain)
  bool attn_force_late_ = false;
  // contexts of at least lm_min_ positions (every step >= 16 splits) merge the splits in a launch of their own
  // (k_attn_merge; graphs g_lm_*); 0: never (QPH_ATTN_MERGE_SEP=0, or too few splits for the context window)
  int lm_min_ = 0, lm_splits_ = 0;
  static constexpr int kLongMergeSplits = 16;
  bool lm_ = false;   // the step being enqueued is such a step
  int pos_ = 0;
  int clean_pos_ = 0;   // the position up to which every enqueued step has been checked clean (see check_status)
  unsigned slot_ = 0;
  hipStream_t st_ = nullptr;
  std::vector<void *> allocs_;
  RansBatch rans_;            // coded (QPACK3) tensors waiting for the load's one decode launch
  RansTiming rans_tm_;
  DMat embed_{}, head_{};
  const float *fnorm_ = nullptr;
  std::vector<Layer> layers_;
  // device state
  float *x_ = nullptr, *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *att_ = nullptr, *h_ = nullptr, *xn_ = nullptr;
  float *logits_ = nullptr, *part_ = nullptr, *cos_ = nullptr, *sin_ = nullptr;
  uint16_t *q16_ = nullptr;   // rotated q as fp16 hi / lo halves (the decode attention's operand)
  float2 *amax_ = nullptr;
  Ctl *ctl_ = nullptr;
  int *out_tok_ = nullptr;
  uint16_t *kc_ = nullptr, *vc_ = nullptr;
  // pinned host
  Ctl *hctl_ = nullptr;
  float *hout_ = nullptr;
  int *htok_ = nullptr;
  // top-M of the logits: device scratch keys, results (values, then indices at kTopkMax) and their pinned host copy
  uint64_t *topk_a_ = nullptr, *topk_b_ = nullptr;
  int *topk_idx_ = nullptr;
  float *topk_val_ = nullptr;
  uint32_t *htopk_ = nullptr;
  int *hstatus_ = nullptr, *dstatus_ = nullptr;   // attention status word: mapped pinned host memory, its device alias
  void topk_to_host(int M, int *idx, float *val);
  hipGraphExec_t g_state_ = nullptr, g_logits_ = nullptr, g_greedy_ = nullptr;
  // decode attention fused with wo (launch_attn_wo) for contexts up to awo_max_ positions (0: not used) and its graphs
  static constexpr int kAwoMaxDefault = 640;   // beyond, split attention + wo is faster (same-box greedy, C3)
  int awo_max_ = 0, awo_rc_ = 0;
  bool awo_rows_ = false;   // the fused kernel is k_attn_wo_rows (every group per workgroup, whole rows, x += y)
  bool fuse_ = false;   // enqueue_layer: the fused kernel (set around a capture or a direct enqueue)
  float *awo_part_ = nullptr;   // [nkv][d] per-group partial wo products
  float *xs_ = nullptr;         // x + the attention block's output (written by the gate / up prologue)
  int *awo_cnt_ = nullptr;      // [row chunks] k_attn_wo arrival counters: its last arrivals add the parts to x
  bool awo_sum_ = false;        // the group parts are added by k_attn_wo (else by the gate / up prologue)
  // the fused graphs per early-load count e = 1..8 (the one-split attention's waves that load their first block before
  // the context is known: ceil(context / 32) up to 8), [e][parts]
  static constexpr int kEarlyMax = 8;
  hipGraphExec_t g_fs_[kEarlyMax + 1][3] = {};
  int early_ = 0;   // enqueue_layer: AttnArgs::early of the fused kernels (set with fuse_)
  hipGraphExec_t g_lm_state_ = nullptr, g_lm_logits_ = nullptr, g_lm_greedy_ = nullptr;
  bool use_graphs_ = true;   // QPH_NO_GRAPH=1: enqueue the kernels directly (profilers that cannot trace graph launches)
  void run_step(int parts, int pos);
  // QPH_GRAPH_STAMPS=file (measurement hook): the graphs are captured with a realtime-stamp region per matvec and
  // k_attn_wo launch, and time_greedy writes the last replayed step's launches (kernel, first start, last end) to file
  struct GStamp { const char *name; size_t off; int n, stride, first, last; };
  static constexpr int kGstWaves = 16384;   // stamp room per matvec launch (waves; its launches have at most ~4K)
  uint64_t *gst_ = nullptr;
  size_t gst_off_ = 0, gst_cap_ = 0;
  bool gst_capturing_ = false;
  std::vector<GStamp> gst_cur_;
  std::vector<std::pair<hipGraphExec_t, std::vector<GStamp>>> gst_graphs_;
  hipGraphExec_t gst_last_ = nullptr;
  uint64_t *gst_take(const char *name, int n, int stride, int first, int last);
  void gst_write(const char *path);
  // reference-order mode (exact.hip)
  int order_ = 0, ex_ncmax_ = 0;
  float *ex_qr_ = nullptr, *ex_part_ = nullptr, *ex_u_ = nullptr, *ex_xn_ = nullptr;
  hipGraphExec_t g_ex_state_ = nullptr, g_ex_logits_ = nullptr, g_ex_greedy_ = nullptr;
  void ex_norm(const float *x, const float *w, float *out, int rows, int ldx);
  void ex_product(const DMat &m, const float *x, int ldx, int ntok, int mm_below, float *y, int ldy, const float *bias,
                  bool resid, bool quantised);
  void ex_enqueue_layer(int l);
  void ex_enqueue_head();
  void ex_prefill(const int *toks, int n);
  void enqueue_step(int parts);
  // batched prompt path (layer matrices q8 / q4)
  static constexpr int kPfChunk = 2048;
  bool pf_ok_ = false;
  int pf_cap_ = 0, pf_ldq_ = 0, pf_ldg_ = 0;
  float *pf_x_ = nullptr, *pf_q_ = nullptr, *pf_k_ = nullptr, *pf_v_ = nullptr, *pf_att_ = nullptr, *pf_g_ = nullptr;
  float *pf_xb_ = nullptr, *pf_xbt_ = nullptr;   // block scales token-major [B][nb], block-major [nb][pf_ldbt_]
  int pf_ldbt_ = 0;
  int8_t *pf_xh_ = nullptr, *pf_xl_ = nullptr;
  int8_t *pf_xh2_ = nullptr, *pf_xl2_ = nullptr;   // second planes: the SwiGLU output quantised by the gate / up store
  float *pf_xb2_ = nullptr, *pf_xbt2_ = nullptr;
  int *pf_tok_ = nullptr, *pf_xg_ = nullptr;
  void prefill_batched(const int *toks, int n);

  void *dalloc(size_t bytes);
  DMat upload(const qph_tensor &t);
  const float *upload_f32(const qph_tensor &t, int64_t n);
  void *place(const void *src, int64_t coded, size_t bytes, const char *name);
  void enqueue_layers();
  void enqueue_layer(int l);
  void qkv_rope(MvArgs &a, uint16_t *kc, uint16_t *vc) const;
  void enqueue_head();
  void build_graphs();
  hipGraphExec_t capture(int parts, bool fused = false, bool long_merge = false, int early = 0);
  // the early-load count of a one-split attention at this position (pos + 1 positions)
  static int early_for(int pos) { return std::min(kEarlyMax, (pos + 1 + 31) / 32); }
  void check_status();
  void write_ctl(int tok, int pos);
};

}  // namespace qph
