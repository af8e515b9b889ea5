#pragma once
// Token sampling from logits: greedy, temperature, top-k, top-p (mirrors
// include/ctd/sampling.h of the reference).
#include <cstdint>
#include <random>
#include <vector>

#include "ctd/tensor.h"

namespace ctd {

struct SamplerConfig {
  float temperature = 1.0f;  // <= 0: greedy (argmax)
  int top_k = 0;             // 0: disabled
  float top_p = 0.0f;        // 0 (or >= 1): disabled
};

// One token per row of logits_last, fp32 [B, 1, V] on the GPU or the host;
// returns the B token ids on the host.  Greedy rows are reduced on the device
// when the logits live there; otherwise each row is drawn on the host with one
// uniform double from rng per row, so a seed fixes the whole token stream.
std::vector<int64_t> sample(const Tensor& logits_last, const SamplerConfig& cfg,
                            std::mt19937_64& rng);

// The host draw for one row of V logits (what sample() runs per row).
int64_t sample_row(const float* logits, int64_t V, const SamplerConfig& cfg,
                   std::mt19937_64& rng);

}  // namespace ctd
