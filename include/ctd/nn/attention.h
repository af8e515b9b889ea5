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
#include "ctd/ops/elementwise.h"
#include "ctd/ops/kv_cache.h"
#include "ctd/ops/mask.h"
#include "ctd/ops/matmul.h"
#include "ctd/ops/permute.h"
#include "ctd/ops/repeat_kv.h"
#include "ctd/ops/rope.h"
#include "ctd/ops/softmax.h"
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

  // The fused attention kernels take head_dim 64 or 128 (every preset);
  // other head sizes run the reference's op chain below.
  static bool fused_head_dim(int D) { return D == 64 || D == 128; }

  // The reference's composition (attention.h:66-91, 123-141 of the
  // reference): Q [B,T,H,D] against Kr, Vr [B,H,L,D], query t seeing keys
  // j <= position_start + t.  Autograd-aware.  -> [B,T,H,D].
  static Tensor attention_chain(const Tensor& Q, const Tensor& Kr, const Tensor& Vr,
                                int position_start, float scale) {
    const int64_t B = Q.shape()[0], T = Q.shape()[1], H = Q.shape()[2], D = Q.shape()[3];
    const int64_t L = Kr.shape()[2];
    Tensor q3 = ops::permute(Q, {0, 2, 1, 3}).reshape({B * H, T, D});
    Tensor s = ops::bmm(q3, Kr.reshape({B * H, L, D}), /*transa=*/false, /*transb=*/true);
    s = ops::apply_causal_mask(ops::mul_scalar(s, scale), position_start);
    Tensor o = ops::bmm(ops::softmax(s), Vr.reshape({B * H, L, D}), false, false);
    return ops::permute(o.reshape({B, H, T, D}), {0, 2, 1, 3});
  }

  // Inference forward (no autograd).  Positions start at position_start.  With
  // kv, this call's K/V go to cache rows [position_start, position_start+T)
  // and the queries attend over rows [0, position_start+T).
  Tensor forward(const Tensor& x, KVLayer* kv = nullptr, int position_start = 0) const {
    return o_proj.forward(forward_context(x, kv, position_start));
  }

  // forward() up to o_proj: the attention output, [B, T, H * D].
  Tensor forward_context(const Tensor& x, KVLayer* kv = nullptr, int position_start = 0) const {
    autograd::NoGradGuard ng;
    const int64_t B = x.shape()[0];
    const int64_t T = x.shape()[1];
    const int H = num_heads, Hk = num_kv_heads, D = head_dim;
    Tensor Q = q_proj.forward(x).reshape({B, T, H, D});
    Tensor K = k_proj.forward(x).reshape({B, T, Hk, D});
    Tensor V = v_proj.forward(x).reshape({B, T, Hk, D});
    if (has_qk_norm()) {
      Q = ops::qk_norm_rope(Q, q_norm.weight, q_norm.eps, position_start, rope_theta,
                            rope_scaling);
      K = ops::qk_norm_rope(K, k_norm.weight, k_norm.eps, position_start, rope_theta,
                            rope_scaling);
    } else {
      ops::apply_rope_inplace(Q, position_start, rope_theta, rope_scaling);
      ops::apply_rope_inplace(K, position_start, rope_theta, rope_scaling);
    }
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    Tensor A;
    if (kv != nullptr) {
      ops::write_kv_inplace(kv->k, K, position_start);
      ops::write_kv_inplace(kv->v, V, position_start);
    }
    if (!fused_head_dim(D)) {
      const int L = kv ? position_start + static_cast<int>(T) : static_cast<int>(T);
      Tensor Kr = kv ? ops::read_kv_expanded(kv->k, L, group())
                     : ops::permute(ops::repeat_kv_heads(K, group()), {0, 2, 1, 3});
      Tensor Vr = kv ? ops::read_kv_expanded(kv->v, L, group())
                     : ops::permute(ops::repeat_kv_heads(V, group()), {0, 2, 1, 3});
      A = attention_chain(Q, Kr, Vr, position_start, scale);
    } else if (position_start == 0) {
      // Prefill: every visible key is one of these T, so the training kernel
      // (MFMA tiles) runs on the fresh projections.
      A = ops::causal_attention_impl(Q, K, V, scale);
    } else if (kv != nullptr) {
      A = ops::cached_attention(Q, kv->k, kv->v, position_start + T, position_start, scale);
    } else {
      A = ops::offset_attention(Q, K, V, position_start, scale);
    }
    return A.reshape({B, T, static_cast<int64_t>(H) * D});
  }

  // Training forward (autograd-aware), positions start at 0.
  Tensor forward_train(const Tensor& x) const { return o_proj.forward(forward_train_context(x)); }

  // forward_train() up to o_proj: the attention output, [B, T, H * D].
  Tensor forward_train_context(const Tensor& x) const {
    const int64_t B = x.shape()[0];
    const int64_t T = x.shape()[1];
    const int H = num_heads, Hk = num_kv_heads, D = head_dim;
    Tensor x2 = q_proj.rows(x);  // one view for the three projections
    Tensor Q = q_proj.forward(x2).reshape({B, T, H, D});
    Tensor K = k_proj.forward(x2).reshape({B, T, Hk, D});
    Tensor V = v_proj.forward(x2).reshape({B, T, Hk, D});
    if (has_qk_norm()) {  // QK-Norm and RoPE in one pass each (bitwise the two ops)
      Q = ops::qk_norm_rope(Q, q_norm.weight, q_norm.eps, 0, rope_theta, rope_scaling);
      K = ops::qk_norm_rope(K, k_norm.weight, k_norm.eps, 0, rope_theta, rope_scaling);
    } else {
      Q = ops::rope(Q, /*position_start=*/0, rope_theta, rope_scaling);
      K = ops::rope(K, /*position_start=*/0, rope_theta, rope_scaling);
    }
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    Tensor A;
    if (fused_head_dim(D)) {
      A = ops::causal_attention(Q, K, V, scale);
    } else {
      Tensor Kr = ops::permute(ops::repeat_kv_heads(K, group()), {0, 2, 1, 3});
      Tensor Vr = ops::permute(ops::repeat_kv_heads(V, group()), {0, 2, 1, 3});
      A = attention_chain(Q, Kr, Vr, 0, scale);
    }
    return A.reshape({B, T, static_cast<int64_t>(H) * D});
  }
};

}  // namespace ctd::nn
