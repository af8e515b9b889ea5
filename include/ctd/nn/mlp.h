#pragma once
// SwiGLU feed-forward: y = down(silu(gate(x)) * up(x)) (mirrors nn/mlp.h of the
// reference); silu and the product run as one fused op.
#include "ctd/autograd.h"
#include "ctd/nn/linear.h"
#include "ctd/ops/elementwise.h"
#include "ctd/tensor.h"

namespace ctd::nn {

struct MLP {
  Linear gate_proj;
  Linear up_proj;
  Linear down_proj;

  Tensor forward(const Tensor& x) const {
    Tensor g = gate_proj.forward(x);
    Tensor u = up_proj.forward(x);
    return down_proj.forward(ops::swiglu(g, u));
  }

  // residual + forward(x), the add done by the down projection's GEMM; gate
  // and up read one [tokens, hidden] view of x.
  Tensor forward_add(const Tensor& x, const Tensor& residual) const {
    return down_proj.forward_add(activation(x), residual);
  }

  // silu(gate(x)) * up(x) as [tokens, intermediate].  With no graph to
  // record (no-grad forward, e.g. the checkpointed forward), the activation
  // overwrites the gate's buffer: one [tokens, intermediate] buffer fewer.
  Tensor activation(const Tensor& x) const {
    Tensor x2 = gate_proj.rows(x);
    Tensor g = gate_proj.forward(x2);
    Tensor u = up_proj.forward(x2);
    if (!autograd::any_requires_grad({g, u})) return ops::swiglu_(g, u);
    return ops::swiglu(g, u);
  }
};

}  // namespace ctd::nn
