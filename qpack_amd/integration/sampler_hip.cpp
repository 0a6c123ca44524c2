// Session-side use of the device top-M (see sampler_hip.hpp).  The arithmetic after the candidate selection restates
// Sampler::dist (/root/reference/src/sampler.cpp:29-57) step for step: it must, since the claim is that the candidate
// route and the logits route give the same distribution bit for bit.
#include "sampler_hip.hpp"

#include <algorithm>
#include <cmath>

namespace qp {
namespace {

// the distinct tokens of the last repeat_last_n entries of history[0, hist_len), in first-seen order (sampler.cpp:32-38)
void penalised(const SamplerParams &p, int V, const std::vector<int> &history, size_t hist_len, std::vector<int> &pen) {
  pen.clear();
  if (p.repeat_penalty == 1.f) return;
  const size_t hn = std::min(hist_len, history.size());
  for (size_t i = hn > (size_t)p.repeat_last_n ? hn - p.repeat_last_n : 0; i < hn; i++) {
    const int t = history[i];
    if (t < 0 || t >= V) continue;
    if (std::find(pen.begin(), pen.end(), t) == pen.end()) pen.push_back(t);
  }
}

int top_k_of(const SamplerParams &p, int V) { return p.temperature <= 0 ? 1 : p.top_k > 0 ? std::min(p.top_k, V) : V; }

constexpr int kDeviceTopM = 512;   // qph_step_topk's largest M

}  // namespace

int hip_topm_size(const SamplerParams &p, int V, const std::vector<int> &history, size_t hist_len) {
  std::vector<int> pen;
  penalised(p, V, history, hist_len, pen);
  const int M = std::min(V, top_k_of(p, V) + (int)pen.size());
  if (M > kDeviceTopM || M >= V / 4) return 0;
  return M;
}

void dist_from_candidates(const SamplerParams &p, int V, std::vector<std::pair<int, float>> cand,
                          const std::vector<int> &history, std::vector<std::pair<int, float>> &out, size_t hist_len) {
  std::vector<int> pen;
  penalised(p, V, history, hist_len, pen);
  const int K = top_k_of(p, V);
  out = std::move(cand);
  for (auto &c : out)
    if (std::find(pen.begin(), pen.end(), c.first) != pen.end())
      c.second = c.second > 0 ? c.second / p.repeat_penalty : c.second * p.repeat_penalty;
  std::sort(out.begin(), out.end(), [](auto &a, auto &b) { return a.second > b.second || (a.second == b.second && a.first < b.first); });
  if ((int)out.size() > K) out.resize(K);
  if (p.temperature <= 0) { out[0].second = 1.f; return; }
  const float mx = out[0].second;
  double sum = 0;
  for (auto &c : out) { c.second = std::exp((c.second - mx) / p.temperature); sum += c.second; }
  size_t keep = out.size();
  double cum = 0;
  for (size_t i = 0; i < out.size(); i++) {
    if (p.min_p > 0 && out[i].second < p.min_p * out[0].second) { keep = std::max<size_t>(i, 1); break; }
    cum += out[i].second / sum;
    if (cum >= p.top_p) { keep = i + 1; break; }
  }
  out.resize(keep);
  double tot = 0;
  for (auto &c : out) tot += c.second;
  for (auto &c : out) c.second = (float)(c.second / tot);
}

int hip_sample_step(Model &m, Sampler &s, int token, const std::vector<int> &history, std::vector<std::pair<int, float>> &dist) {
  const SamplerParams &p = s.params();
  const int V = m.vocab();
  const int M = hip_topm_size(p, V, history);
  std::vector<std::pair<int, float>> cand;
  if (M > 0 && hip_step_candidates(m, token, M, cand)) {
    dist_from_candidates(p, V, std::move(cand), history, dist);
  } else {
    const float *l = m.step(token, 1);
    s.dist(l, V, history, dist);
  }
  return s.draw(dist);
}

}  // namespace qp
