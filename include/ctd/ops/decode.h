#pragma once
// Fused ops for decode steps (a few token rows): each streams its weights once
// and folds the small ops around it into the same kernel.  Not in the
// reference, whose decode runs the per-module ops (include/ctd/nn/
// transformer_block.h:17-24); TransformerBlock::forward uses these when a KV
// cache is given and the call has at most kDecodeMaxRows token rows.
#include <vector>

#include "ctd/ops/rope.h"
#include "ctd/tensor.h"

namespace ctd::ops {

constexpr int64_t kDecodeMaxRows = 8;

// For each weight W_i [N_i, K]: y_i = W_i xn (+ residuals[i] when given, same
// shape as y_i), xn = RMSNorm(x; norm_w, eps) when norm_w is defined, else x.
// x [..., K] with at most kDecodeMaxRows rows; y_i [..., N_i].  1 to 3 weights.
std::vector<Tensor> decode_linear(const Tensor& x, const Tensor& norm_w, float eps,
                                  const std::vector<Tensor>& weights,
                                  const std::vector<Tensor>& residuals = {});

// silu(W_gate xn) * (W_up xn), xn as above: the MLP's input half.  -> [..., I].
Tensor decode_gate_up(const Tensor& x, const Tensor& norm_w, float eps, const Tensor& w_gate,
                      const Tensor& w_up);

// q [B,T,H*D], k/v [B,T,Hk*D]: per-head QK-Norm (when q_norm_w / k_norm_w are
// defined), RoPE from position_start, k and v written to the cache rows
// [position_start, position_start+T) of k_cache / v_cache [B,Hk,S,D].
// Returns the rotated q [B,T,H,D].
Tensor decode_qkv_post(const Tensor& q, const Tensor& k, const Tensor& v, int num_heads,
                       int num_kv_heads, int head_dim, const Tensor& q_norm_w,
                       const Tensor& k_norm_w, float eps, float theta, const RopeScaling& scaling,
                       int position_start, Tensor& k_cache, Tensor& v_cache);

// decode_qkv_post followed by cached_attention(q, k_cache, v_cache,
// position_start + T, position_start, scale), in one launch (plus the split
// merge).  Returns the attention output [B,T,H,D].
Tensor decode_qkv_attention(const Tensor& q, const Tensor& k, const Tensor& v, int num_heads,
                            int num_kv_heads, int head_dim, const Tensor& q_norm_w,
                            const Tensor& k_norm_w, float eps, float theta,
                            const RopeScaling& scaling, int position_start, Tensor& k_cache,
                            Tensor& v_cache, float scale);

}  // namespace ctd::ops
