#pragma once
// Softmax along the last axis (mirrors ops/softmax.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

Tensor softmax(const Tensor& x);
Tensor softmax_impl(const Tensor& x);
// dx = y * (g - sum(g * y, -1))
Tensor softmax_backward_impl(const Tensor& y, const Tensor& g);

}  // namespace ctd::ops
