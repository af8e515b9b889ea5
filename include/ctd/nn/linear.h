#pragma once
// Linear layer without bias: y = x W^T (mirrors nn/linear.h of the reference).
#include <stdexcept>

#include "ctd/ops/matmul.h"
#include "ctd/tensor.h"

namespace ctd::nn {

struct Linear {
  Tensor weight;  // [out, in]

  Tensor forward(const Tensor& x) const {
    const int64_t in = weight.shape()[1];
    const int64_t out = weight.shape()[0];
    const auto& sh = x.shape();
    if (sh.back() != in) throw std::runtime_error("Linear: in_features mismatch");
    const int64_t leading = x.numel() / in;
    Tensor y2d = ops::matmul(x.reshape({leading, in}), weight, /*transa=*/false, /*transb=*/true);
    std::vector<int64_t> out_shape(sh.begin(), sh.end());
    out_shape.back() = out;
    return y2d.reshape(out_shape);
  }

  // residual + forward(x) as one GEMM whose store does the add (bitwise equal
  // to the two ops, same backward); residual has forward(x)'s shape.
  Tensor forward_add(const Tensor& x, const Tensor& residual) const {
    const int64_t in = weight.shape()[1];
    const int64_t out = weight.shape()[0];
    const auto& sh = x.shape();
    if (sh.back() != in) throw std::runtime_error("Linear: in_features mismatch");
    const int64_t leading = x.numel() / in;
    std::vector<int64_t> out_shape(sh.begin(), sh.end());
    out_shape.back() = out;
    if (residual.shape() != out_shape)
      throw std::runtime_error("Linear: residual shape mismatch");
    Tensor y2d = ops::matmul_add(x.reshape({leading, in}), weight, /*transa=*/false,
                                 /*transb=*/true, residual.reshape({leading, out}));
    return y2d.reshape(out_shape);
  }

  // forward(x)'s autograd graph without the product: the result is a view of
  // `values` (forward(x)'s shape).  See ops::matmul_graph_only.
  Tensor forward_graph_only(const Tensor& x, const Tensor& values) const {
    const int64_t in = weight.shape()[1];
    const int64_t out = weight.shape()[0];
    const auto& sh = x.shape();
    if (sh.back() != in) throw std::runtime_error("Linear: in_features mismatch");
    const int64_t leading = x.numel() / in;
    Tensor y2d = ops::matmul_graph_only(x.reshape({leading, in}), weight, /*transa=*/false,
                                        /*transb=*/true, values);
    std::vector<int64_t> out_shape(sh.begin(), sh.end());
    out_shape.back() = out;
    return y2d.reshape(out_shape);
  }
};

}  // namespace ctd::nn
