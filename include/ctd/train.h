#pragma once
// The training-step driver of the reference's `ctd_train` tool
// (tools/ctd_train/main.cpp), as a library: JSON run config, the pre-tokenised
// binary data format, warmup + cosine learning rate, gradient accumulation,
// clipping, loss.jsonl logging, validation, and checkpoint save / resume with
// the optimizer state.  `emberlm_amd/lib/ctd_train --config <path>` runs it.

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
// prefetch (nn::Model::recompute_hook -> optim::AdamW::prefetch): layer 1,
// the second-to-last one the backward re-runs, so that two layers of
// backward cover the transfer of the embedding's m/v (2.55 GB, about 45 ms,
// at Qwen3-1.7B; 2.15 GB against 2 x 26 ms of backward at LLaMA-3.2-1B,
// B=4, T=2048).  Models of one layer get no prefetch.
constexpr int kOptimizerPrefetchLayer = 1;

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
