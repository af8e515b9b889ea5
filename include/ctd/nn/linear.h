#pragma once
// Linear layer without bias: y = x W^T (mirrors nn/linear.h of the reference).
#include <stdexcept>

#include "ctd/ops/matmul.h"
#include "ctd/tensor.h"

namespace ctd::nn {

struct Linear {
  Tensor weight;  // [out, in]

  Tensor forward(const Tensor& x) const {
    return shaped(ops::matmul(rows(x), weight, /*transa=*/false, /*transb=*/true), out_shape(x));
  }

  // residual + forward(x) as one GEMM whose store does the add (bitwise equal
  // to the two ops, same backward); residual has forward(x)'s elements and
  // shapes the result.
  Tensor forward_add(const Tensor& x, const Tensor& residual) const {
    const int64_t out = weight.shape()[0];
    Tensor x2 = rows(x);
    if (residual.shape().back() != out || residual.numel() != x2.shape()[0] * out)
      throw std::runtime_error("Linear: residual shape mismatch");
    Tensor r2 = residual.dim() == 2 ? residual : residual.reshape({x2.shape()[0], out});
    return shaped(ops::matmul_add(x2, weight, /*transa=*/false, /*transb=*/true, r2),
                  residual.shape());
  }

  // forward(x)'s autograd graph without the product: the result is a view of
  // `values` (forward(x)'s elements).  See ops::matmul_graph_only.
  Tensor forward_graph_only(const Tensor& x, const Tensor& values) const {
    return shaped(ops::matmul_graph_only(rows(x), weight, /*transa=*/false, /*transb=*/true,
                                         values),
                  out_shape(x));
  }

  // x as [leading, in_features]: x itself when it is 2-D already, so that
  // projections of one input share its node and their input gradients meet
  // in one place (where the engine adds them inside the second GEMM).
  Tensor rows(const Tensor& x) const {
    const int64_t in = weight.shape()[1];
    if (x.shape().back() != in) throw std::runtime_error("Linear: in_features mismatch");
    return x.dim() == 2 ? x : x.reshape({x.numel() / in, in});
  }

 private:
  std::vector<int64_t> out_shape(const Tensor& x) const {
    std::vector<int64_t> sh(x.shape().begin(), x.shape().end());
    sh.back() = weight.shape()[0];
    return sh;
  }
  static Tensor shaped(const Tensor& y2d, const std::vector<int64_t>& shape) {
    return y2d.shape() == shape ? y2d : y2d.reshape(shape);
  }
};

}  // namespace ctd::nn
