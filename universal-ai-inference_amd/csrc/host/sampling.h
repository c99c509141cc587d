// sampling.h — token selection from a scores row (libs/uaii-runtime/src/sampling.cpp:22-125).
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

#include "error.h"

namespace uaii {
namespace runtime {

// include/uaii/runtime/sampling.hpp:15-27.
struct SampleParams {
  float temperature = 0.0f;
  float top_p = 1.0f;               // nucleus; 1.0 = off
  int32_t top_k = 0;                // 0 = off
  float repetition_penalty = 1.0f;  // 1.0 = off; > 1 penalises ids in `penalty_tokens`
  uint64_t seed = 0;
  bool has_seed = false;
  bool greedy() const noexcept {
    return temperature <= 0.0f && top_k <= 0 && top_p >= 1.0f - 1e-6f &&
           repetition_penalty <= 1.0f + 1e-6f;
  }
};

// Pick one id from row[0..vocab): greedy argmax (strict '>', lowest index wins)
// when params.greedy(), else repetition penalty, temperature, top-k, softmax,
// top-p and one uniform draw from *rng, in the reference's order and with the
// same standard-library selection, sort and distribution, so the same row, params
// and generator state give the same id.
Error sample_token_f32(const float* row, size_t vocab, const SampleParams& params,
                       const std::vector<int64_t>& penalty_tokens, std::mt19937_64* rng,
                       int64_t* out_token);

}  // namespace runtime
}  // namespace uaii
