#pragma once
// Elementwise ops (mirrors ops/elementwise.h of the reference) plus the fused
// SwiGLU used by nn::MLP.
#include "ctd/tensor.h"

namespace ctd::ops {

Tensor add(const Tensor& a, const Tensor& b);
Tensor add_impl(const Tensor& a, const Tensor& b);
// add()'s backward node without the sum: a view of `values` (a's shape, left
// as they are) carrying that node; see matmul_graph_only.  Added in this build.
Tensor add_graph_only(const Tensor& a, const Tensor& b, const Tensor& values);
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
// g = silu(g) * u in place, returning g; records no graph and throws when g or
// u requires grad.  For callers that own g and read it no more (nn::MLP under
// no-grad, where the gate's buffer then holds the activation).  Added in this
// build.
Tensor swiglu_(Tensor& g, const Tensor& u);

}  // namespace ctd::ops
