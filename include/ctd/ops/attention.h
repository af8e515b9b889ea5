#pragma once
// Fused causal GQA attention.  Computes exactly what the reference's chain
// bmm -> mul_scalar -> apply_causal_mask -> softmax -> bmm (with
// repeat_kv_heads and permutes, include/ctd/nn/attention.h:123-141 of the
// reference) computes, without materialising the [B*H, T, T] scores.
#include "ctd/tensor.h"

namespace ctd::ops {

// q [B,T,H,D], k/v [B,T,Hk,D] -> o [B,T,H,D]; H % Hk == 0, D in {64, 128}.
// Autograd-aware: saves q, k, v, o and the per-row log-sum-exp.
Tensor causal_attention(const Tensor& q, const Tensor& k, const Tensor& v, float scale);
// Forward only; lse (if non-null) receives the [B,H,T] log-sum-exp.
Tensor causal_attention_impl(const Tensor& q, const Tensor& k, const Tensor& v, float scale,
                             Tensor* lse = nullptr);

}  // namespace ctd::ops
