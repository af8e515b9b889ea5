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
// passes (ember_attn_bwd_scattered): less than a layer's full dS splits the
// pass into chunks of KV rows (one (batch, KV head) pair each), 0 recomputes
// dS in the dQ pass instead; -1 restores the default
// (kAttentionBackwardDsBytes).  Results do not depend on it.  The default
// holds half the dS of a Qwen3-1.7B layer at B=8, T=4096 (32 of 64 KV rows
// of 68 MB: two chunks).  The rows are spread over up to 16 free blocks the
// device allocator already holds, and the backward keeps fewer rows (in
// equal chunks) rather than grow the memory held: it grows it only when the
// free blocks hold fewer than 16 rows, and then only to 16.  All 64 rows
// (one chunk) ran the layer's backward 0.25 ms faster (10.83 against 11.08
// ms) but would raise the step's live peak from 21.8 to 23.3 GB: the
// attention backward starts at 18.9 GB live.
constexpr int64_t kAttentionBackwardDsBytes = 2500000000;
void set_attention_backward_ds_bytes(int64_t bytes);
// Added in this build (off by default): a causal_attention whose inputs
// require grad keeps its scores S = Q K^T (fp32, the causal part, 4.36 GB per
// Qwen3-1.7B layer at B=8, T=4096) from the forward to its backward, which then
// reads them instead of computing S again (4 of the 5 products it runs
// otherwise) and writes dS over them.  Meant for a checkpointed block's re-run,
// whose backward follows at once; every other forward that records a graph
// holds its scores until its backward too.  The buffers come from the device
// allocator's free blocks (up to 16 pieces, grown if need be); with a retained
// graph the backward computes S again and leaves the scores intact.  dQ, dK
// and dV agree with the default path to fp32 rounding.
void set_attention_keep_scores(bool on);
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
