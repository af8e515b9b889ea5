#pragma once
// Embedding lookup and deterministic backward (mirrors ops/embedding.h of the reference).
#include "ctd/tensor.h"

namespace ctd::ops {

// ids int64 [...], weight fp32 [vocab, hidden] -> fp32 [..., hidden]
Tensor embedding(const Tensor& ids, const Tensor& weight);
Tensor embedding_impl(const Tensor& ids, const Tensor& weight);
// dW[id, :] = sum of dy rows with that id (fresh dense [vocab, hidden]).
Tensor embedding_backward_impl(const Tensor& ids, const Tensor& dy, int64_t vocab);
// dw[id, :] += the same row sums, into an existing [vocab, hidden] tensor
// (a tied weight's running gradient).  Added in this build.
void embedding_backward_into(const Tensor& ids, const Tensor& dy, Tensor& dw);

}  // namespace ctd::ops
