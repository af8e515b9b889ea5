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

// Inference attention with a position offset (no autograd): query t of q
// [B,T,H,D] sees keys j <= position_start + t among the first valid_len rows of
// a KV cache k/v [B,Hk,S,D] (the reference's read_kv_expanded -> bmm ->
// mul_scalar -> apply_causal_mask(position_start) -> softmax -> bmm,
// include/ctd/nn/attention.h:66-91).  -> o [B,T,H,D].
Tensor cached_attention(const Tensor& q, const Tensor& k_cache, const Tensor& v_cache,
                        int64_t valid_len, int position_start, float scale);
// The same over k/v [B,T,Hk,D] projections (no cache; valid_len = T).
Tensor offset_attention(const Tensor& q, const Tensor& k, const Tensor& v, int position_start,
                        float scale);

}  // namespace ctd::ops
