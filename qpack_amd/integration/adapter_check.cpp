// Check harness for the reference-side binding: links the same objects as the reference's qpack-bench build (the
// reference's sources, the qp::Model adapter, the load_model branch, the device-sampler glue) and drives them the way
// the reference's callers do.  tests/test_integration.py runs it.
//
//   adapter_check greedy MODEL N TOK...     load_model (QPACK_DEVICE picks the backend), prefill(TOK..., want 1), then
//                                           greedy_run from the prompt's argmax for N tokens; prints arch, file size,
//                                           the first token and the stream
//   adapter_check sample MODEL STEPS TOP_K PENALTY TEMP SEED TOK...
//                                           after prefill(TOK...), per step: the next token sampled three ways from the
//                                           same position - Sampler::dist on step(tok, 1)'s logits, dist_from_candidates
//                                           on the device top-M, and hip_sample_step - with three samplers of one seed;
//                                           the distributions must be equal bit for bit and the draws the same token
//   adapter_check candidates-cpu SEED       no model: dist_from_candidates on a host top-M (a full sort) against
//                                           Sampler::dist on random logits with ties, several parameter sets
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "qpack/engine.h"
#include "qpack/qpack.h"
#include "sampler_hip.hpp"

using Dist = std::vector<std::pair<int, float>>;

static bool same_bits(const Dist &a, const Dist &b) {
  if (a.size() != b.size()) return false;
  for (size_t i = 0; i < a.size(); i++)
    if (a[i].first != b[i].first || memcmp(&a[i].second, &b[i].second, 4)) return false;
  return true;
}

// the M best (index, value) pairs, value descending and the lower index first: what top_m selects, by a full sort
static Dist host_top_m(const float *x, int V, int M) {
  Dist all((size_t)V);
  for (int v = 0; v < V; v++) all[(size_t)v] = {v, x[v]};
  std::sort(all.begin(), all.end(), [](auto &a, auto &b) { return a.second > b.second || (a.second == b.second && a.first < b.first); });
  all.resize((size_t)M);
  return all;
}

static int greedy(const char *path, int n, const std::vector<int> &prompt) {
  auto m = qp::load_model(path, (int)prompt.size() + n + 8);
  const float *l = m->prefill(prompt.data(), (int)prompt.size(), 1);
  const int first = (int)(std::max_element(l, l + m->vocab()) - l);
  std::vector<int> out((size_t)n);
  const int got = m->greedy_run(first, n, out.data());
  printf("arch %s\nfile_size %zu\nfirst %d\ngreedy", m->arch().c_str(), m->container().file_size(), first);
  for (int i = 0; i < got; i++) printf(" %d", out[(size_t)i]);
  printf("\n");
  return got == n ? 0 : 1;
}

static int sample(const char *path, int steps, qp::SamplerParams p, const std::vector<int> &prompt) {
  auto m = qp::load_model(path, (int)prompt.size() + steps + 8);
  const int V = m->vocab();
  qp::Sampler s_logits(p), s_cand(p), s_step(p);
  std::vector<int> hist = prompt;
  const float *l = m->prefill(prompt.data(), (int)prompt.size(), 1);
  int tok = (int)(std::max_element(l, l + V) - l);   // the first fed token: the prompt's argmax
  int bad = 0, device_steps = 0;
  for (int i = 0; i < steps; i++) {
    hist.push_back(tok);
    const int pos0 = m->pos();
    Dist d_logits, d_cand, d_step;
    const float *lg = m->step(tok, 1);
    s_logits.dist(lg, V, hist, d_logits);
    const int t_logits = s_logits.draw(d_logits);
    const int M = qp::hip_topm_size(p, V, hist);
    int t_cand = t_logits;
    if (M > 0) {
      if (!m->rewind(pos0)) { fprintf(stderr, "rewind failed\n"); return 2; }
      Dist cand;
      if (!qp::hip_step_candidates(*m, tok, M, cand)) { fprintf(stderr, "not a HIP model\n"); return 2; }
      qp::dist_from_candidates(p, V, cand, hist, d_cand);
      t_cand = s_cand.draw(d_cand);
      device_steps++;
    } else {
      d_cand = d_logits; s_cand.draw(d_cand);
    }
    if (!m->rewind(pos0)) { fprintf(stderr, "rewind failed\n"); return 2; }
    const int t_step = qp::hip_sample_step(*m, s_step, tok, hist, d_step);
    const bool ok = same_bits(d_logits, d_cand) && same_bits(d_logits, d_step) && t_logits == t_cand && t_logits == t_step;
    if (!ok) bad++;
    printf("step %d M %d n %zu token %d %d %d %s\n", i, M, d_logits.size(), t_logits, t_cand, t_step, ok ? "same" : "DIFFERENT");
    tok = t_logits;
  }
  printf("device_steps %d different %d\n", device_steps, bad);
  return bad ? 1 : 0;
}

static int candidates_cpu(uint64_t seed) {
  std::mt19937_64 rng(seed);
  const int V = 151936;
  std::vector<float> x((size_t)V);
  std::normal_distribution<float> nd(0.f, 3.f);
  int bad = 0, cases = 0;
  for (int rep = 0; rep < 24; rep++) {
    for (auto &v : x) v = nd(rng);
    // ties and signed zeros among the largest values, which the order's index rule decides
    for (int k = 0; k < 40; k++) x[(size_t)(rng() % V)] = 9.5f;
    x[(size_t)(rng() % V)] = 0.f; x[(size_t)(rng() % V)] = -0.f;
    if (rep % 3 == 2) for (int k = 0; k < 200; k++) x[(size_t)(rng() % V)] = -0.f;
    std::vector<int> hist;
    for (int k = 0; k < 100; k++) hist.push_back((int)(rng() % V));
    for (int k = 0; k < 20; k++) hist.push_back((int)(std::max_element(x.begin(), x.end()) - x.begin()));
    const int ks[] = {1, 40, 448, 512};
    for (int K : ks)
      for (float pen : {1.f, 1.1f, 0.9f})
        for (float temp : {0.f, 0.7f, 1.3f}) {
          qp::SamplerParams p; p.top_k = K; p.repeat_penalty = pen; p.temperature = temp; p.seed = seed + rep;
          p.top_p = rep % 2 ? 0.9f : 1.f; p.min_p = rep % 4 < 2 ? 0.05f : 0.f;
          const int M = qp::hip_topm_size(p, V, hist);
          if (!M) continue;
          qp::Sampler a(p), b(p);
          Dist da, db;
          a.dist(x.data(), V, hist, da);
          qp::dist_from_candidates(p, V, host_top_m(x.data(), V, M), hist, db);
          cases++;
          if (!same_bits(da, db) || a.draw(da) != b.draw(db)) { bad++; printf("differ: rep %d K %d pen %g temp %g\n", rep, K, pen, temp); }
        }
  }
  printf("cases %d different %d\n", cases, bad);
  return bad || cases < 100 ? 1 : 0;
}

int main(int argc, char **argv) {
  try {
    if (argc >= 4 && !strcmp(argv[1], "greedy")) {
      std::vector<int> prompt;
      for (int i = 4; i < argc; i++) prompt.push_back(atoi(argv[i]));
      return greedy(argv[2], atoi(argv[3]), prompt);
    }
    if (argc >= 9 && !strcmp(argv[1], "sample")) {
      qp::SamplerParams p;
      p.top_k = atoi(argv[4]); p.repeat_penalty = (float)atof(argv[5]); p.temperature = (float)atof(argv[6]);
      p.seed = strtoull(argv[7], nullptr, 10);
      std::vector<int> prompt;
      for (int i = 8; i < argc; i++) prompt.push_back(atoi(argv[i]));
      return sample(argv[2], atoi(argv[3]), p, prompt);
    }
    if (argc == 3 && !strcmp(argv[1], "candidates-cpu")) return candidates_cpu(strtoull(argv[2], nullptr, 10));
  } catch (std::exception &e) {
    fprintf(stderr, "error: %s\n", e.what());
    return 3;
  }
  fprintf(stderr, "usage: adapter_check greedy MODEL N TOK... | sample MODEL STEPS TOP_K PENALTY TEMP SEED TOK... | candidates-cpu SEED\n");
  return 2;
}
