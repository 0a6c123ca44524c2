// Sampling on the HIP model from the device's top-M candidates instead of the full logits: the Session-side half of
// the device sampler.  Sampler::dist (/root/reference/src/sampler.cpp:29-57) begins with top_m(logits, V, K + |pen|)
// (:12-27), the M largest (index, value) pairs under the order value descending, lower index first; the device top-M
// (qph_step_topk) returns exactly that set in exactly that order, so everything after top_m runs unchanged on it and
// the distribution, and the token Sampler::draw picks from it, are the same bits as from the full logits.
#pragma once
#include <utility>
#include <vector>

#include "qpack/engine.h"
#include "qpack/qpack.h"

namespace qp {

// The M that Sampler::dist would pass to top_m for these parameters and this history (K + the distinct penalised
// tokens), or 0 when the device top-M cannot stand in for top_m: M above 512 (the device selection's limit), or
// M >= V / 4, where top_m takes all V entries instead of the M largest.
int hip_topm_size(const SamplerParams &p, int V, const std::vector<int> &history, size_t hist_len = (size_t)-1);

// Sampler::dist from its line 41 on (penalties, sort, top-k cut, temperature, min-p / top-p, normalisation), with the
// top_m result `cand` in place of the logits.  `cand` must be what top_m would return for M = hip_topm_size(...).
void dist_from_candidates(const SamplerParams &p, int V, std::vector<std::pair<int, float>> cand,
                          const std::vector<int> &history, std::vector<std::pair<int, float>> &out,
                          size_t hist_len = (size_t)-1);

// The device top-M step of a model made by make_llama_hip: feeds `token`, returns the M best (index, value) pairs
// of the next logits in `cand`.  false (nothing fed) when `m` is not a HIP model.
bool hip_step_candidates(Model &m, int token, int M, std::vector<std::pair<int, float>> &cand);

// What Session::generate's plain decoding does per token (/root/reference/src/chat.cpp:219, next_token at :207-211):
// feed `token`, then sample the next one with `s`.  `history` already ends with `token`.  On a HIP model whose
// sampler parameters allow it (hip_topm_size > 0) only the device's top-M crosses PCIe; otherwise
// the logits are taken (want = 1) and Sampler::dist runs on them.  Either way the result is the same token.
int hip_sample_step(Model &m, Sampler &s, int token, const std::vector<int> &history, std::vector<std::pair<int, float>> &dist);

}  // namespace qp
