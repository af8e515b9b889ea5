#pragma once
// Multi-head attention with GQA, RoPE (+llama3 scaling), optional QK-Norm and
// a causal mask (mirrors nn/attention.h of the reference).  forward_train keeps
// Q/K/V in their projection layout [B,T,H,D] and calls the fused causal
// attention op, so nothing of size [B*H,T,T] and no repeat_kv/permute copies
// are created.
#include <cmath>
#include <stdexcept>

#include "ctd/nn/linear.h"
#include "ctd/nn/rms_norm.h"
#include "ctd/ops/attention.h"
#include "ctd/ops/rope.h"
#include "ctd/tensor.h"

namespace ctd::nn {

struct Attention {
  Linear q_proj;
  Linear k_proj;
  Linear v_proj;
  Linear o_proj;
  int num_heads = 0;
  int num_kv_heads = 0;
  int head_dim = 0;
  float rope_theta = 100000.0f;
  ops::RopeScaling rope_scaling{};

  // QK-Norm (Qwen3): RMSNorm over head_dim on Q and K before RoPE; skipped when
  // the weight is empty.
  RMSNorm q_norm{Tensor{}, 0.0f};
  RMSNorm k_norm{Tensor{}, 0.0f};
  bool has_qk_norm() const { return q_norm.weight.storage() != nullptr; }

  int group() const { return num_heads / num_kv_heads; }
  int hidden_size() const { return num_heads * head_dim; }

  // Training forward (autograd-aware), positions start at 0.
  Tensor forward_train(const Tensor& x) const {
    const int64_t B = x.shape()[0];
    const int64_t T = x.shape()[1];
    const int H = num_heads, Hk = num_kv_heads, D = head_dim;
    Tensor Q = q_proj.forward(x).reshape({B, T, H, D});
    Tensor K = k_proj.forward(x).reshape({B, T, Hk, D});
    Tensor V = v_proj.forward(x).reshape({B, T, Hk, D});
    if (has_qk_norm()) {
      Q = q_norm.forward(Q);
      K = k_norm.forward(K);
    }
    Q = ops::rope(Q, /*position_start=*/0, rope_theta, rope_scaling);
    K = ops::rope(K, /*position_start=*/0, rope_theta, rope_scaling);
    Tensor A = ops::causal_attention(Q, K, V, 1.0f / std::sqrt(static_cast<float>(D)));
    return o_proj.forward(A.reshape({B, T, static_cast<int64_t>(H) * D}));
  }
};

}  // namespace ctd::nn
