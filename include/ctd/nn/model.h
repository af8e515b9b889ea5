#pragma once
// LlamaConfig presets, Model and weight loading (mirrors nn/model.h of the reference).
#include <functional>
#include <string>
#include <vector>

#include "ctd/autograd.h"
#include "ctd/nn/embedding.h"
#include "ctd/nn/kv_cache.h"
#include "ctd/nn/linear.h"
#include "ctd/nn/rms_norm.h"
#include "ctd/nn/transformer_block.h"
#include "ctd/ops/loss.h"
#include "ctd/safetensors.h"
#include "ctd/tensor.h"

namespace ctd::nn {

struct LlamaConfig {
  int vocab_size;
  int hidden_size;
  int intermediate_size;
  int num_hidden_layers;
  int num_attention_heads;
  int num_key_value_heads;
  int head_dim;
  int max_position_embeddings;
  float rms_norm_eps;
  float rope_theta;
  bool tie_word_embeddings;
  bool qk_norm = false;
  float rope_scaling_factor = 0.0f;
  float rope_scaling_low_freq_factor = 1.0f;
  float rope_scaling_high_freq_factor = 4.0f;
  int rope_scaling_original_max_pos = 8192;
};

LlamaConfig smollm2_135m_config();
LlamaConfig smollm2_360m_config();
LlamaConfig qwen3_0_6b_config();
LlamaConfig qwen3_1_7b_config();
LlamaConfig llama3_2_1b_config();

// Picks a preset from the embed_tokens shape (hidden size, vocab).
LlamaConfig autodetect_config(const TensorDict& w);
inline LlamaConfig autodetect_smollm2_config(const TensorDict& w) { return autodetect_config(w); }

struct Model {
  LlamaConfig config{};
  Embedding embed_tokens;
  std::vector<TransformerBlock> layers;
  RMSNorm norm;
  bool gradient_checkpointing = false;
  // Called with the layer index when the backward pass re-runs a checkpointed
  // layer's forward, before the re-run (never during the forward pass itself).
  // A trainer uses it to start work that should overlap the end of the
  // backward, such as staging the offloaded optimizer state
  // (optim::AdamW::prefetch).  Empty: nothing is called.
  std::function<void(int)> recompute_hook;

  // Inference: input_ids int64 [B, T] -> logits fp32 [B, T, vocab], positions
  // from position_start.  With a cache, each layer's K/V are written at rows
  // [position_start, position_start+T) and cache->current_len becomes
  // position_start + T.
  Tensor forward(const Tensor& input_ids, KVCache* cache = nullptr,
                 int position_start = 0) const;
  // The same forward, but the LM head runs on the last position of each row
  // only: logits [B, 1, vocab] (what a sampler consumes).
  Tensor forward_last_logits(const Tensor& input_ids, KVCache* cache = nullptr,
                             int position_start = 0) const;
  // input_ids int64 [B, T] -> logits fp32 [B, T, vocab]
  Tensor forward_train_logits(const Tensor& input_ids) const;
  // Mean cross-entropy over all positions, shape [1].
  Tensor forward_train(const Tensor& input_ids, const Tensor& targets) const;
  // SFT loss with fp32 loss_mask [B, T].
  Tensor forward_train_masked(const Tensor& input_ids, const Tensor& targets,
                              const Tensor& loss_mask) const;

  struct NamedParameters {
    std::vector<std::pair<std::string, Tensor>> all;
    std::vector<Tensor> decay;
    std::vector<Tensor> no_decay;
    std::vector<std::string> decay_names;
    std::vector<std::string> no_decay_names;
  };
  // Marks every parameter requires_grad and splits decay / no_decay in the
  // reference's order (embed, per layer: norms, projections, ..., final norm).
  NamedParameters collect_parameters();
};

// Builds a Model from HF-named weights (model.embed_tokens.weight, model.layers.{i}...).
Model build_model(const TensorDict& w, const LlamaConfig& cfg);

}  // namespace ctd::nn
