// Model presets, forward paths, HF-named weight loading and parameter grouping.
// Reference: include/ctd/nn/model.h:19-217 and src/nn/model.cpp:24-100.
#include "ctd/nn/model.h"

#include <stdexcept>
#include <string>

#include "ctd/ops/decode.h"
#include "ctd/ops/loss.h"
#include "ctd/runtime.h"
#include "ember_hip.h"

namespace ctd::nn {

LlamaConfig smollm2_135m_config() {
  LlamaConfig c{};
  c.vocab_size = 49152;
  c.hidden_size = 576;
  c.intermediate_size = 1536;
  c.num_hidden_layers = 30;
  c.num_attention_heads = 9;
  c.num_key_value_heads = 3;
  c.head_dim = 64;
  c.max_position_embeddings = 8192;
  c.rms_norm_eps = 1e-5f;
  c.rope_theta = 100000.0f;
  c.tie_word_embeddings = true;
  return c;
}

LlamaConfig smollm2_360m_config() {
  LlamaConfig c = smollm2_135m_config();
  c.hidden_size = 960;
  c.intermediate_size = 2560;
  c.num_hidden_layers = 32;
  c.num_attention_heads = 15;
  c.num_key_value_heads = 5;
  return c;
}

LlamaConfig qwen3_0_6b_config() {
  LlamaConfig c{};
  c.vocab_size = 151936;
  c.hidden_size = 1024;
  c.intermediate_size = 3072;
  c.num_hidden_layers = 28;
  c.num_attention_heads = 16;
  c.num_key_value_heads = 8;
  c.head_dim = 128;
  c.max_position_embeddings = 40960;
  c.rms_norm_eps = 1e-6f;
  c.rope_theta = 1000000.0f;
  c.tie_word_embeddings = true;
  c.qk_norm = true;
  return c;
}

LlamaConfig qwen3_1_7b_config() {
  LlamaConfig c = qwen3_0_6b_config();
  c.hidden_size = 2048;
  c.intermediate_size = 6144;
  return c;
}

LlamaConfig llama3_2_1b_config() {
  LlamaConfig c{};
  c.vocab_size = 128256;
  c.hidden_size = 2048;
  c.intermediate_size = 8192;
  c.num_hidden_layers = 16;
  c.num_attention_heads = 32;
  c.num_key_value_heads = 8;
  c.head_dim = 64;
  c.max_position_embeddings = 131072;
  c.rms_norm_eps = 1e-5f;
  c.rope_theta = 500000.0f;
  c.tie_word_embeddings = true;
  c.qk_norm = false;
  c.rope_scaling_factor = 32.0f;
  c.rope_scaling_low_freq_factor = 1.0f;
  c.rope_scaling_high_freq_factor = 4.0f;
  c.rope_scaling_original_max_pos = 8192;
  return c;
}

LlamaConfig autodetect_config(const TensorDict& w) {
  auto it = w.find("model.embed_tokens.weight");
  if (it == w.end()) throw std::runtime_error("autodetect_config: missing model.embed_tokens.weight");
  const int64_t vocab = it->second.shape().at(0);
  const int64_t hidden = it->second.shape().at(1);
  if (hidden == 576) return smollm2_135m_config();
  if (hidden == 960) return smollm2_360m_config();
  if (hidden == 1024 && vocab == 151936) return qwen3_0_6b_config();
  if (hidden == 2048 && vocab == 151936) return qwen3_1_7b_config();
  if (hidden == 2048 && vocab == 128256) return llama3_2_1b_config();
  throw std::runtime_error("autodetect_config: unsupported hidden_size=" + std::to_string(hidden) +
                           " vocab_size=" + std::to_string(vocab));
}

namespace {

// Hidden states [B, T, H] after the last block of the inference forward
// (model.h:152-163 of the reference, before the final norm and the LM head).
Tensor hidden_states(const Model& m, const Tensor& input_ids, KVCache* cache,
                     int position_start) {
  if (input_ids.dim() != 2) throw std::runtime_error("Model::forward: input_ids must be [B, T]");
  if (cache) {
    if (cache->layers.size() != m.layers.size())
      throw std::runtime_error("Model::forward: KV cache has " +
                               std::to_string(cache->layers.size()) + " layers, model has " +
                               std::to_string(m.layers.size()));
    if (cache->batch != input_ids.shape()[0])
      throw std::runtime_error("Model::forward: KV cache batch != input batch");
  }
  Tensor h = m.embed_tokens.forward(input_ids);
  for (size_t i = 0; i < m.layers.size(); ++i) {
    KVLayer* kv = cache ? &cache->layers[i] : nullptr;
    h = m.layers[i].forward(h, kv, position_start);
  }
  if (cache) cache->current_len = position_start + input_ids.shape()[1];
  return h;
}

}  // namespace

Tensor Model::forward(const Tensor& input_ids, KVCache* cache, int position_start) const {
  autograd::NoGradGuard ng;
  Tensor h = norm.forward(hidden_states(*this, input_ids, cache, position_start));
  Linear lm_head{embed_tokens.weight};  // tied head
  return lm_head.forward(h);
}

Tensor Model::forward_last_logits(const Tensor& input_ids, KVCache* cache,
                                  int position_start) const {
  autograd::NoGradGuard ng;
  Tensor h = hidden_states(*this, input_ids, cache, position_start);
  const int64_t B = h.shape()[0], T = h.shape()[1], H = h.shape()[2];
  Tensor last;
  if (B == 1) {
    last = h.view_at((T - 1) * H, {1, 1, H});
  } else {
    last = Tensor::empty({B, 1, H}, DType::kFloat32, h.device());
    for (int64_t b = 0; b < B; ++b)
      CTD_CHECK(ember_memcpy_async(static_cast<float*>(last.data_ptr()) + b * H,
                                   static_cast<const float*>(h.data_ptr()) + (b * T + T - 1) * H,
                                   H * sizeof(float), 2, runtime::compute_stream()));
  }
  if (B <= ops::kDecodeMaxRows)  // final RMSNorm folded into the LM-head GEMV
    return ops::decode_linear(last, norm.weight, norm.eps, {embed_tokens.weight})[0];
  Linear lm_head{embed_tokens.weight};
  return lm_head.forward(norm.forward(last));
}

namespace {

// embedding -> blocks (checkpointed when enabled) -> final RMSNorm: [B, T, H].
Tensor train_hidden(const Model& m, const Tensor& input_ids) {
  Tensor h = m.embed_tokens.forward(input_ids);
  for (size_t i = 0; i < m.layers.size(); ++i) {
    const TransformerBlock& layer = m.layers[i];
    if (m.gradient_checkpointing) {
      // checkpoint() runs fn under no-grad in the forward pass and with grad
      // enabled when the backward pass re-runs it; the re-run only
      // back-propagates through its result, so the block skips computing it.
      const int li = static_cast<int>(i);
      h = autograd::checkpoint(
          [&m, &layer, li](const Tensor& x) {
            if (!autograd::is_grad_enabled()) return layer.forward_train(x);
            if (m.recompute_hook) m.recompute_hook(li);
            return layer.forward_train_for_backward(x);
          },
          h);
    } else {
      h = layer.forward_train(h);
    }
  }
  return m.norm.forward(h);
}

}  // namespace

Tensor Model::forward_train_logits(const Tensor& input_ids) const {
  Linear lm_head{embed_tokens.weight};  // tied head
  return lm_head.forward(train_hidden(*this, input_ids));
}

// The losses run the tied LM head and the cross-entropy together a chunk of
// rows at a time (ops::linear_cross_entropy_masked): the same loss as
// cross_entropy(forward_train_logits(...)) without the [B*T, V] logits.
Tensor Model::forward_train(const Tensor& input_ids, const Tensor& targets) const {
  const int64_t total = input_ids.numel();
  Tensor h = train_hidden(*this, input_ids);
  Tensor ones = Tensor::empty({total}, DType::kFloat32, h.device());
  CTD_CHECK(ember_fill(static_cast<float*>(ones.data_ptr()), total, 1.0f,
                       runtime::compute_stream()));
  return ops::linear_cross_entropy_masked(h.reshape({total, h.shape().back()}),
                                          embed_tokens.weight, targets.reshape({total}), ones);
}

Tensor Model::forward_train_masked(const Tensor& input_ids, const Tensor& targets,
                                   const Tensor& loss_mask) const {
  const int64_t total = input_ids.numel();
  Tensor h = train_hidden(*this, input_ids);
  return ops::linear_cross_entropy_masked(h.reshape({total, h.shape().back()}),
                                          embed_tokens.weight, targets.reshape({total}),
                                          loss_mask.reshape({total}));
}

namespace {

// The weights of one decoder layer as data: the HF key under
// "model.layers.<i>.", whether AdamW decays it (the projections) or not (the
// norms), whether it exists only in QK-Norm models, and the block member that
// holds it.  The row order is collect_parameters' order within a layer, which
// fixes the checkpoint's tensor order and the optimizer-state layout
// (src/nn/model.cpp:63-100 of the reference lists the same keys in the same
// order).
struct LayerWeight {
  const char* key;
  bool decay;
  bool qk_norm_only;
  Tensor& (*slot)(TransformerBlock&);
};

constexpr LayerWeight kLayerWeights[] = {
    {"input_layernorm.weight", false, false,
     [](TransformerBlock& b) -> Tensor& { return b.input_layernorm.weight; }},
    {"self_attn.q_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.self_attn.q_proj.weight; }},
    {"self_attn.k_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.self_attn.k_proj.weight; }},
    {"self_attn.v_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.self_attn.v_proj.weight; }},
    {"self_attn.o_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.self_attn.o_proj.weight; }},
    {"self_attn.q_norm.weight", false, true,
     [](TransformerBlock& b) -> Tensor& { return b.self_attn.q_norm.weight; }},
    {"self_attn.k_norm.weight", false, true,
     [](TransformerBlock& b) -> Tensor& { return b.self_attn.k_norm.weight; }},
    {"post_attention_layernorm.weight", false, false,
     [](TransformerBlock& b) -> Tensor& { return b.post_attention_layernorm.weight; }},
    {"mlp.gate_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.mlp.gate_proj.weight; }},
    {"mlp.up_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.mlp.up_proj.weight; }},
    {"mlp.down_proj.weight", true, false,
     [](TransformerBlock& b) -> Tensor& { return b.mlp.down_proj.weight; }},
};

constexpr const char* kEmbedKey = "model.embed_tokens.weight";  // also the tied LM head
constexpr const char* kFinalNormKey = "model.norm.weight";

std::string layer_prefix(size_t i) { return "model.layers." + std::to_string(i) + "."; }

const Tensor& required(const TensorDict& w, const std::string& key) {
  auto it = w.find(key);
  if (it == w.end()) throw std::runtime_error("build_model: the weights have no tensor " + key);
  return it->second;
}

}  // namespace

Model build_model(const TensorDict& w, const LlamaConfig& cfg) {
  Model m;
  m.config = cfg;
  m.embed_tokens.weight = required(w, kEmbedKey);
  m.norm = RMSNorm{required(w, kFinalNormKey), cfg.rms_norm_eps};
  const ops::RopeScaling scaling{cfg.rope_scaling_factor, cfg.rope_scaling_low_freq_factor,
                            cfg.rope_scaling_high_freq_factor, cfg.rope_scaling_original_max_pos};
  m.layers.resize(static_cast<size_t>(cfg.num_hidden_layers));
  for (size_t i = 0; i < m.layers.size(); ++i) {
    TransformerBlock& blk = m.layers[i];
    Attention& a = blk.self_attn;
    a.num_heads = cfg.num_attention_heads;
    a.num_kv_heads = cfg.num_key_value_heads;
    a.head_dim = cfg.head_dim;
    a.rope_theta = cfg.rope_theta;
    a.rope_scaling = scaling;
    for (RMSNorm* n : {&blk.input_layernorm, &blk.post_attention_layernorm, &a.q_norm, &a.k_norm})
      n->eps = cfg.rms_norm_eps;
    const std::string pre = layer_prefix(i);
    for (const LayerWeight& lw : kLayerWeights) {
      auto it = w.find(pre + lw.key);
      if (it != w.end())
        lw.slot(blk) = it->second;
      else if (!lw.qk_norm_only)
        required(w, pre + lw.key);  // throws
    }
  }
  return m;
}

Model::NamedParameters Model::collect_parameters() {
  NamedParameters out;
  auto take = [&out](std::string name, Tensor& t, bool decay) {
    t.requires_grad_(true);
    (decay ? out.decay : out.no_decay).push_back(t);
    (decay ? out.decay_names : out.no_decay_names).push_back(name);
    out.all.emplace_back(std::move(name), t);
  };
  take(kEmbedKey, embed_tokens.weight, true);
  for (size_t i = 0; i < layers.size(); ++i) {
    const std::string pre = layer_prefix(i);
    for (const LayerWeight& lw : kLayerWeights) {
      Tensor& t = lw.slot(layers[i]);
      if (lw.qk_norm_only && !t.defined()) continue;
      take(pre + lw.key, t, lw.decay);
    }
  }
  take(kFinalNormKey, norm.weight, false);
  return out;
}

}  // namespace ctd::nn
