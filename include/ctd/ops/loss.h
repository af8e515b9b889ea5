#pragma once
// Cross-entropy losses (mirrors ops/loss.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// logits fp32 [N, V], targets int64 [N] -> scalar [1] = mean over rows.
Tensor cross_entropy(const Tensor& logits, const Tensor& targets);
Tensor cross_entropy_impl(const Tensor& logits, const Tensor& targets);

// loss = sum_i mask_i * (-log p_i[t_i]) / sum_i mask_i; throws in backward if
// sum(mask) == 0.
Tensor cross_entropy_masked(const Tensor& logits, const Tensor& targets,
                            const Tensor& loss_mask);
Tensor cross_entropy_masked_impl(const Tensor& logits, const Tensor& targets,
                                 const Tensor& loss_mask);

}  // namespace ctd::ops
