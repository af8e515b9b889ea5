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

// d + matmul(a, b, transa, transb) in one GEMM (the add done as the product
// is stored, bitwise equal to the two ops), with both ops' backward nodes:
// the residual connections of a block.  d is [M, N] contiguous.  Added in
// this build; the reference runs matmul and then ops::add.
Tensor matmul_add(const Tensor& a, const Tensor& b, bool transa, bool transb, const Tensor& d);

// Batched matmul: a [B, Ma, Ka], b [B, Mb, Kb] -> [B, M, N].
Tensor bmm(const Tensor& a, const Tensor& b, bool transa = false, bool transb = false);
Tensor bmm_impl(const Tensor& a, const Tensor& b, bool transa, bool transb);

}  // namespace ctd::ops
