#pragma once
// Causal attention mask (mirrors ops/mask.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

void apply_causal_mask_inplace(Tensor& scores, int q_pos_start = 0);
Tensor apply_causal_mask(const Tensor& scores, int q_pos_start = 0);
Tensor apply_causal_mask_impl(const Tensor& scores, int q_pos_start);
Tensor causal_mask_backward_impl(const Tensor& g, int q_pos_start);

}  // namespace ctd::ops
