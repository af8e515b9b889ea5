#pragma once
// RMSNorm (mirrors ops/norm.h of the reference).
#include <utility>

#include "ctd/tensor.h"

namespace ctd::ops {

// y = x * rsqrt(mean(x^2, -1) + eps) * weight; backward gives grads for x and weight.
Tensor rms_norm(const Tensor& x, const Tensor& weight, float eps);
Tensor rms_norm_impl(const Tensor& x, const Tensor& weight, float eps);
std::pair<Tensor, Tensor> rms_norm_backward_impl(const Tensor& dy, const Tensor& x,
                                                 const Tensor& w, float eps);

}  // namespace ctd::ops
