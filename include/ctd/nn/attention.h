#pragma once
// Multi-head attention with GQA, RoPE (+llama3 scaling), optional QK-Norm, a
// causal mask and a KV cache (mirrors nn/attention.h of the reference).  Both
// forwards keep Q/K/V in their projection layout [B,T,H,D] and call fused
// attention kernels, so nothing of size [B*H,T,L] and no repeat_kv/permute
// copies are created.
#include <cmath>
#include <stdexcept>

#include "ctd/autograd.h"
#include "ctd/nn/kv_cache.h"
#include "ctd/nn/linear.h"
#include "ctd/nn/rms_norm.h"
#include "ctd/ops/attention.h"
#include "ctd/ops/kv_cache.h"
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

  // Inference forward (no autograd).  Positions start at position_start.  With
  // kv, this call's K/V go to cache rows [position_start, position_start+T)
  // and the queries attend over rows [0, position_start+T).
  Tensor forward(const Tensor& x, KVLayer* kv = nullptr, int position_start = 0) const {
    autograd::NoGradGuard ng;
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
    ops::apply_rope_inplace(Q, position_start, rope_theta, rope_scaling);
    ops::apply_rope_inplace(K, position_start, rope_theta, rope_scaling);
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    Tensor A;
    if (kv != nullptr) {
      ops::write_kv_inplace(kv->k, K, position_start);
      ops::write_kv_inplace(kv->v, V, position_start);
    }
    if (position_start == 0) {
      // Prefill: every visible key is one of these T, so the training kernel
      // (MFMA tiles) runs on the fresh projections.
      A = ops::causal_attention_impl(Q, K, V, scale);
    } else if (kv != nullptr) {
      A = ops::cached_attention(Q, kv->k, kv->v, position_start + T, position_start, scale);
    } else {
      A = ops::offset_attention(Q, K, V, position_start, scale);
    }
    return o_proj.forward(A.reshape({B, T, static_cast<int64_t>(H) * D}));
  }

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
