#pragma once
// Elementwise ops (mirrors ops/elementwise.h of the reference) plus the fused
// SwiGLU used by nn::MLP.
#include "ctd/tensor.h"

namespace ctd::ops {

Tensor add(const Tensor& a, const Tensor& b);
Tensor add_impl(const Tensor& a, const Tensor& b);
Tensor mul(const Tensor& a, const Tensor& b);
Tensor mul_impl(const Tensor& a, const Tensor& b);
// SiLU: y = x * sigmoid(x).
Tensor silu(const Tensor& x);
Tensor silu_impl(const Tensor& x);

Tensor sub_impl(const Tensor& a, const Tensor& b);
Tensor scale_impl(const Tensor& x, float alpha);
// d(silu)/dx * g
Tensor silu_backward_impl(const Tensor& x, const Tensor& g);

// h = silu(g) * u in one pass; saves g and u, recomputes silu(g) in backward.
Tensor swiglu(const Tensor& g, const Tensor& u);
Tensor swiglu_impl(const Tensor& g, const Tensor& u);

}  // namespace ctd::ops
