// sampling.cpp — host token selection for non-greedy SampleParams.
//
// Follows libs/uaii-runtime/src/sampling.cpp:22-125 step by step: the kept
// candidates' order after std::nth_element / std::sort decides which id a
// uniform draw lands on, so the same standard-library algorithms are used on the
// same (value, id) pairs with the same comparator. Greedy selection never comes
// here from the device token loop (the argmax runs on the GPU).
#include "sampling.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <utility>

#pragma clang fp contract(off)

namespace uaii {
namespace runtime {
namespace {

// HF-style repetition penalty (sampling.cpp:14-18): positive logits divided,
// negative ones multiplied.
inline float penalised(float v, float penalty, bool seen) {
  if (!seen || penalty <= 1.0f + 1e-6f) return v;
  return v > 0.0f ? v / penalty : v * penalty;
}

}  // namespace

Error sample_token_f32(const float* row, size_t vocab, const SampleParams& params,
                       const std::vector<int64_t>& penalty_tokens, std::mt19937_64* rng,
                       int64_t* out_token) {
  if (row == nullptr || out_token == nullptr)
    return Error::make(ErrorCode::InvalidArgument, "sample_token null");
  if (vocab == 0) return Error::make(ErrorCode::InvalidArgument, "sample_token empty vocab");

  std::vector<char> seen(vocab, 0);
  for (int64_t t : penalty_tokens)
    if (t >= 0 && (size_t)t < vocab) seen[(size_t)t] = 1;
  const float pen = params.repetition_penalty;

  if (params.greedy()) {
    size_t best = 0;
    float bv = penalised(row[0], pen, seen[0] != 0);
    for (size_t i = 1; i < vocab; ++i) {
      const float v = penalised(row[i], pen, seen[i] != 0);
      if (v > bv) { bv = v; best = i; }
    }
    *out_token = (int64_t)best;
    return Error::success();
  }
  if (rng == nullptr) return Error::make(ErrorCode::InvalidArgument, "sample_token requires rng");

  using Cand = std::pair<float, int64_t>;
  const auto higher = [](const Cand& a, const Cand& b) { return a.first > b.first; };
  std::vector<Cand> c;
  c.reserve(vocab);
  const float inv_t = 1.0f / std::max(params.temperature, 1e-5f);
  for (size_t i = 0; i < vocab; ++i) c.emplace_back(penalised(row[i], pen, seen[i] != 0) * inv_t, (int64_t)i);

  // top-k: the k largest, in nth_element's arrangement
  if (params.top_k > 0 && (size_t)params.top_k < c.size()) {
    const size_t k = (size_t)params.top_k;
    std::nth_element(c.begin(), c.begin() + (std::ptrdiff_t)k, c.end(), higher);
    c.resize(k);
  }

  // softmax over the kept values (max-shifted; the sum runs in kept order)
  float mx = -std::numeric_limits<float>::infinity();
  for (const Cand& e : c) mx = std::max(mx, e.first);
  float sum = 0.0f;
  for (Cand& e : c) {
    e.first = std::exp(e.first - mx);
    sum += e.first;
  }
  if (!(sum > 0.0f) || !std::isfinite(sum)) {
    auto it = std::max_element(c.begin(), c.end(), [](const Cand& a, const Cand& b) { return a.first < b.first; });
    *out_token = it->second;
    return Error::success();
  }
  for (Cand& e : c) e.first /= sum;

  // top-p: descending probabilities, keep through the first that reaches top_p
  if (params.top_p > 0.0f && params.top_p < 1.0f - 1e-6f) {
    std::sort(c.begin(), c.end(), higher);
    float cum = 0.0f;
    size_t keep = 0;
    for (; keep < c.size(); ++keep) {
      cum += c[keep].first;
      if (cum >= params.top_p) {
        ++keep;
        break;
      }
    }
    if (keep == 0) keep = 1;
    c.resize(keep);
    float renorm = 0.0f;
    for (const Cand& e : c) renorm += e.first;
    if (renorm > 0.0f)
      for (Cand& e : c) e.first /= renorm;
  }

  std::uniform_real_distribution<float> unit(0.0f, 1.0f);
  const float r = unit(*rng);
  float cum = 0.0f;
  for (const Cand& e : c) {
    cum += e.first;
    if (r <= cum) {
      *out_token = e.second;
      return Error::success();
    }
  }
  *out_token = c.back().second;
  return Error::success();
}

}  // namespace runtime
}  // namespace uaii
