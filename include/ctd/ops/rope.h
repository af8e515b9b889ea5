#pragma once
// Rotary position embedding, non-interleaved (mirrors ops/rope.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// LLaMA 3 frequency scaling. factor <= 1 means vanilla RoPE.
struct RopeScaling {
  float factor = 0.0f;
  float low_freq_factor = 1.0f;
  float high_freq_factor = 4.0f;
  int original_max_pos = 8192;

  bool enabled() const { return factor > 1.0f; }
  float low_freq_wavelen() const { return static_cast<float>(original_max_pos) / low_freq_factor; }
  float high_freq_wavelen() const {
    return static_cast<float>(original_max_pos) / high_freq_factor;
  }
};

// x: fp32 [B, T, H, D], D even.
void apply_rope_inplace(Tensor& x, int position_start, float theta,
                        const RopeScaling& scaling = {});
Tensor rope(const Tensor& x, int position_start, float theta, const RopeScaling& scaling = {});
Tensor rope_impl(const Tensor& x, int position_start, float theta,
                 const RopeScaling& scaling = {});
Tensor rope_transpose_impl(const Tensor& x, int position_start, float theta,
                           const RopeScaling& scaling = {});

// rope(rms_norm(x, weight, eps), ...) with one backward node: x [B, T, H, D]
// normalised over D per head (QK-Norm) and rotated, in one pass when D is 64
// or 128 (bitwise the two ops), by the two ops otherwise.  Added in this
// build; the reference runs RMSNorm::forward and then rope.
Tensor qk_norm_rope(const Tensor& x, const Tensor& weight, float eps, int position_start,
                    float theta, const RopeScaling& scaling = {});

}  // namespace ctd::ops
