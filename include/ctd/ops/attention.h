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
// Device memory the backward may use to keep dS between its dK/dV and dQ
// passes (ember_attn_bwd): less than a layer's full dS splits the pass into
// chunks of KV heads, 0 recomputes dS in the dQ pass instead; -1 restores the
// default (kAttentionBackwardDsBytes).  Results do not depend on it.  The
// default holds Qwen3-1.7B's dS at B=8, T=4096 (4.4 GB per layer) in four
// chunks, and the backward takes less than that when the device allocator
// holds no free block that large but one of at least half of it.  A budget of
// 2.5 GB (two chunks) ran 0.67 ms per layer faster there, but no block that
// size stays free among the checkpoints and gradients of a step, so the
// allocator grew by 2.4 GB at a time and held 1.32x the live bytes (1.10x at
// this default); smaller models fit in one or two chunks.
constexpr int64_t kAttentionBackwardDsBytes = 1250000000;
void set_attention_backward_ds_bytes(int64_t bytes);
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
