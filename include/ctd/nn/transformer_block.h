#pragma once
// Llama-style decoder block: h = x + attn(norm(x)); y = h + mlp(norm(h))
// (mirrors nn/transformer_block.h of the reference).
#include "ctd/nn/attention.h"
#include "ctd/nn/mlp.h"
#include "ctd/nn/rms_norm.h"
#include "ctd/ops/decode.h"
#include "ctd/ops/elementwise.h"
#include "ctd/tensor.h"

namespace ctd::nn {

struct TransformerBlock {
  RMSNorm input_layernorm;
  RMSNorm post_attention_layernorm;
  Attention self_attn;
  MLP mlp;

  // Inference forward.  With a KV cache and at most ops::kDecodeMaxRows token
  // rows (a decode step), the fused decode kernels run the same functions in
  // five launches (six when long contexts split the keys); otherwise the
  // module ops run one by one.
  Tensor forward(const Tensor& x, KVLayer* kv = nullptr, int position_start = 0) const {
    autograd::NoGradGuard ng;
    if (kv != nullptr && x.dim() == 3 && x.shape()[0] * x.shape()[1] <= ops::kDecodeMaxRows &&
        Attention::fused_head_dim(self_attn.head_dim))
      return decode_step(x, *kv, position_start);
    Tensor h1 = input_layernorm.forward(x);
    Tensor h = self_attn.o_proj.forward_add(self_attn.forward_context(h1, kv, position_start), x);
    Tensor h2 = post_attention_layernorm.forward(h);
    return mlp.forward_add(h2, h);
  }

  Tensor decode_step(const Tensor& x, KVLayer& kv, int position_start) const {
    const int64_t B = x.shape()[0], T = x.shape()[1];
    const Attention& at = self_attn;
    const int H = at.num_heads, Hk = at.num_kv_heads, D = at.head_dim;
    auto qkv = ops::decode_linear(x, input_layernorm.weight, input_layernorm.eps,
                                  {at.q_proj.weight, at.k_proj.weight, at.v_proj.weight});
    Tensor a = ops::decode_qkv_attention(qkv[0], qkv[1], qkv[2], H, Hk, D, at.q_norm.weight,
                                         at.k_norm.weight, at.q_norm.eps, at.rope_theta,
                                         at.rope_scaling, position_start, kv.k, kv.v,
                                         1.0f / std::sqrt(static_cast<float>(D)));
    Tensor h = ops::decode_linear(a.reshape({B, T, static_cast<int64_t>(H) * D}), Tensor{}, 0.0f,
                                  {at.o_proj.weight}, {x})[0];
    Tensor m = ops::decode_gate_up(h, post_attention_layernorm.weight,
                                   post_attention_layernorm.eps, mlp.gate_proj.weight,
                                   mlp.up_proj.weight);
    return ops::decode_linear(m, Tensor{}, 0.0f, {mlp.down_proj.weight}, {h})[0];
  }

  // The residual adds run inside the o_proj and down_proj GEMMs (bitwise the
  // same as ops::add after the product, same autograd graph).
  Tensor forward_train(const Tensor& x) const {
    Tensor h1 = input_layernorm.forward(x);
    Tensor h = self_attn.o_proj.forward_add(self_attn.forward_train_context(h1), x);
    Tensor h2 = post_attention_layernorm.forward(h);
    return mlp.forward_add(h2, h);
  }

  // forward_train(x) for a checkpoint's recompute, whose backward reads only
  // the graph of the block's output: down_proj and the last residual add are
  // recorded but not run, so the returned tensor has forward_train(x)'s
  // grad_fn but no values of its own (a placeholder: data_ptr() and
  // copy_to_host() throw).  Its gradients are forward_train's, kernel for
  // kernel.  The checkpointed forward already computed the real output: it is
  // the next block's saved input.
  Tensor forward_train_for_backward(const Tensor& x) const {
    Tensor h1 = input_layernorm.forward(x);
    Tensor h = self_attn.o_proj.forward_add(self_attn.forward_train_context(h1), x);
    Tensor h2 = post_attention_layernorm.forward(h);
    Tensor m = mlp.down_proj.forward_graph_only(mlp.activation(h2), h);
    return ops::add_graph_only(h, m.reshape(h.shape()), h).mark_placeholder();
  }
};

}  // namespace ctd::nn
