// sampler.cpp -- the host temperature / top-p sampler (mcpm_sample_logits);
// the engine's sampled decode runs the device sampler (mcpm_sampler.hip).
//
// Sampler::sample (src/sampler.cpp:8-73): optional temperature scaling,
// softmax with the max subtracted, probabilities sorted in decreasing order,
// cut at cumulative top_p and renormalised, then the first token whose
// running sum reaches a uniform draw.  The reference seeds std::mt19937 from
// std::random_device (src/sampler.cpp:5-6); here the caller passes the seed.
// Equal probabilities are ordered by token id (std::sort leaves that order
// unspecified).
#include <algorithm>
#include <random>
#include <vector>

#include "mcpm_host.h"

namespace mcpm {

int sample_token(const float* logits, int n, float temperature, float top_p, float r) {
  const float inv_temp = (temperature > 0.0f) ? (1.0f / temperature) : 1.0f;
  const bool apply_temp = (temperature != 1.0f && temperature > 0.0f);
  float maxl = -1e9f;
  for (int i = 0; i < n; ++i) {
    const float v = apply_temp ? logits[i] * inv_temp : logits[i];
    if (v > maxl) maxl = v;
  }
  std::vector<std::pair<float, int>> pr(n);
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    const float v = apply_temp ? logits[i] * inv_temp : logits[i];
    pr[i] = {exp_f32(v - maxl), i};
    sum = sum + pr[i].first;
  }
  for (int i = 0; i < n; ++i) pr[i].first = pr[i].first / sum;
  size_t cnt = pr.size();
  if (top_p > 0.0f && top_p < 1.0f) {
    std::sort(pr.begin(), pr.end(), [](const std::pair<float, int>& a, const std::pair<float, int>& b) {
      return a.first > b.first || (a.first == b.first && a.second < b.second);
    });
    float cum = 0.0f;
    size_t last = 0;
    for (size_t i = 0; i < pr.size(); ++i) {
      cum = cum + pr[i].first;
      last = i;
      if (cum >= top_p) break;
    }
    cnt = last + 1;
    for (size_t i = 0; i < cnt; ++i) pr[i].first = pr[i].first / cum;
  }
  float cur = 0.0f;
  for (size_t i = 0; i < cnt; ++i) {
    cur = cur + pr[i].first;
    if (r <= cur) return pr[i].second;
  }
  return pr[cnt - 1].second;
}

}  // namespace mcpm

extern "C" int mcpm_sample_logits(const float* logits, int n, float temperature, float top_p, float r) {
  if (!logits || n <= 0) return mcpm::fail(MCPM_ERR_ARG, "mcpm_sample_logits: bad argument");
  return mcpm::sample_token(logits, n, temperature, top_p, r);
}
