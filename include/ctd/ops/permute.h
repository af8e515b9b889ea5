#pragma once
// Axis permutation (mirrors ops/permute.h of the reference).
#include <vector>

#include "ctd/tensor.h"

namespace ctd::ops {

// New contiguous tensor with y.shape[i] = x.shape[perm[i]]; rank <= 6.
Tensor permute(const Tensor& x, const std::vector<int>& perm);
Tensor permute_impl(const Tensor& x, const std::vector<int>& perm);

}  // namespace ctd::ops
