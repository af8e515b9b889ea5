#pragma once
// Matrix multiply on the fp32 MFMA GEMM (mirrors ops/matmul.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// 2D matmul with optional transpose flags. Autograd-aware.
Tensor matmul(const Tensor& a, const Tensor& b, bool transa = false, bool transb = false);
Tensor matmul_impl(const Tensor& a, const Tensor& b, bool transa, bool transb);

// The backward node matmul(a, b, transa, transb) records, without computing
// the product: the result is a view of `values` (M*N contiguous floats, left
// as they are) carrying that node.  For a product that only the backward pass
// reaches, e.g. a checkpointed block's output during its recompute.  Added in
// this build; the reference has no counterpart.
Tensor matmul_graph_only(const Tensor& a, const Tensor& b, bool transa, bool transb,
                         const Tensor& values);

// Batched matmul: a [B, Ma, Ka], b [B, Mb, Kb] -> [B, M, N].
Tensor bmm(const Tensor& a, const Tensor& b, bool transa = false, bool transb = false);
Tensor bmm_impl(const Tensor& a, const Tensor& b, bool transa, bool transb);

}  // namespace ctd::ops
