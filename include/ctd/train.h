#pragma once
// The training-step driver of the reference's `ctd_train` tool
// (tools/ctd_train/main.cpp), as a library: JSON run config, the pre-tokenised
// binary data format, warmup + cosine learning rate, gradient accumulation,
// clipping, loss.jsonl logging, validation, and checkpoint save / resume with
// the optimizer state.  `emberlm_amd/lib/ctd_train --config <path>` runs it.

#include <cmath>
#include <cstdint>
#include <filesystem>
#include <string>
#include <vector>

#include "ctd/nn/model.h"
#include "ctd/optim.h"
#include "ctd/tensor.h"

namespace ctd::train {

// Run config (main.cpp:46-101); unset keys keep these defaults.
struct Config {
  std::string run_name;
  std::filesystem::path run_dir;  // the config file's directory
  std::filesystem::path init_weights;
  std::filesystem::path resume_from;
  std::filesystem::path data_dir;
  int seq_len = 1024;
  int batch_size = 1;
  int grad_accum_steps = 8;
  int total_steps = 2800;
  int warmup_steps = 100;
  float lr = 3e-4f;
  float min_lr_ratio = 0.1f;
  float weight_decay = 0.1f;
  float beta1 = 0.9f;
  float beta2 = 0.95f;
  float eps = 1e-8f;
  float clip_grad_norm = 1.0f;
  int val_every = 100;
  int save_every = 500;
  int log_every = 1;
  uint64_t seed = 42;
  bool offload_optimizer = false;
  bool gradient_checkpointing = false;
  // Optional "model" object (not in the reference, which only autodetects its
  // presets from the embedding shape): LlamaConfig fields by name, for shapes
  // autodetection does not know, e.g. small test models.
  bool has_model = false;
  nn::LlamaConfig model{};
};

// Parses the JSON config; init_weights and data_dir are required.
Config load_config(const std::filesystem::path& cfg_path);

// A model architecture from a JSON file holding the fields of the config's
// "model" object (HF config names: vocab_size, hidden_size, ...).
nn::LlamaConfig load_model_config(const std::filesystem::path& path);

// One split of the pre-tokenised data (main.cpp:115-136): `<split>.bin` holds
// int32 token ids, seq_len per document; `<split>_mask.bin` one int8 loss-mask
// value per token.
struct DataSplit {
  std::vector<int32_t> tokens;
  std::vector<int8_t> masks;
  int64_t num_docs = 0;
};
DataSplit load_split(const std::filesystem::path& tok_path,
                     const std::filesystem::path& mask_path, int seq_len);

// Host side of a batch (main.cpp:145-168): for each picked document, inputs
// are tokens [0, seq_len-1), targets tokens [1, seq_len), and the mask of a
// position is the mask value of its target token.
struct HostBatch {
  std::vector<int64_t> input_ids, targets;
  std::vector<float> loss_mask;
  float sum_mask = 0.0f;
  int64_t B = 0, T = 0;  // T = seq_len - 1
};
HostBatch make_host_batch(const DataSplit& split, const std::vector<int64_t>& doc_indices,
                          int seq_len);

struct Batch {
  Tensor input_ids, targets, loss_mask;
  float sum_mask = 0.0f;
};
Batch make_batch(const DataSplit& split, const std::vector<int64_t>& doc_indices, int seq_len,
                 Device device);

// Linear warmup to c.lr, then cosine decay to c.lr * c.min_lr_ratio at
// total_steps (main.cpp:176-188), in float as there.
float lr_at_step(int step, const Config& c);

// Layer whose re-run in the backward pass starts the offloaded optimizer's
// prefetch (nn::Model::recompute_hook -> optim::AdamW::prefetch) for a batch
// of `tokens`, or -1 for no prefetch.  The backward of that layer and of the
// ones below it should cover the prefetch's copies, the embedding's m and v
// (8 V d bytes) at about 50 GB/s, so that step() need not wait for them.  A
// layer's backward re-runs its forward and runs its own, about 6 x tokens x
// (its parameters) flops, estimated at 130 TFLOP/s.  Only a lead of one or
// two layers is used, where the prefetch pays for its staging buffer
// (Qwen3-1.7B at B=8, T=4096: layer 1, step 4045 -> 4006 ms for +0.8 GB of
// peak HBM; LLaMA-3.2-1B at B=4, T=2048: layer 2, 828 -> 771 ms).  Models
// that would need more lead have short forwards that wait little for the
// update (Qwen3-0.6B at B=4, T=1024, layer 9: 278 -> 276 ms for a peak of
// 6.12 -> 6.75 GB; SmolLM2-135M, layer 14: 105.5 -> 105.1 ms).
inline int optimizer_prefetch_layer(const nn::LlamaConfig& c, int64_t tokens) {
  constexpr double kMaxLead = 2.0;
  const double d = c.hidden_size, D = c.head_dim;
  const double layer_params = d * D * (2.0 * c.num_attention_heads + 2.0 * c.num_key_value_heads) +
                              3.0 * d * c.intermediate_size;
  const double layer_s = 6.0 * static_cast<double>(tokens) * layer_params / 130e12;
  const double copy_s = 8.0 * c.vocab_size * d / 50e9;
  const double k = layer_s > 0.0 ? std::ceil(copy_s / layer_s) : kMaxLead + 1.0;
  if (k > kMaxLead || static_cast<int>(k) > c.num_hidden_layers - 1) return -1;
  return k < 1.0 ? 1 : static_cast<int>(k);
}

// Mask-weighted mean masked CE over the whole split, one document per forward
// (main.cpp:191-206).
float run_val(const nn::Model& model, const DataSplit& val, int seq_len, Device device);

// Optimizer state next to a weights checkpoint: `<weights>.opt.safetensors`
// with optimizer.m.<name> / optimizer.v.<name> (decay group first) and
// optimizer.step (main.cpp:208-271).  Loading writes offloaded state straight
// into its pinned host buffers.
std::filesystem::path opt_path_for(const std::filesystem::path& weights_path);
void save_optimizer_state(optim::AdamW& opt, const nn::Model::NamedParameters& named,
                          const std::filesystem::path& path);
void load_optimizer_state(optim::AdamW& opt, const nn::Model::NamedParameters& named,
                          const std::filesystem::path& path);

// One loss.jsonl record of a training step: keys grad_norm, loss, lr, phase,
// step, tokens_per_sec, wall_s (sorted, as the reference's JSON library
// writes them).
std::string train_event(int step, float loss, float lr, float grad_norm, double tokens_per_sec,
                        double wall_s);
// A validation record: keys loss, phase, step, wall_s.
std::string val_event(int step, float loss, double wall_s);

// The whole ctd_train run (main.cpp:275-431).  Returns 0 on success; errors
// throw std::runtime_error.
int run(const Config& cfg);

}  // namespace ctd::train
