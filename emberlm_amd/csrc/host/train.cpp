// Training-step driver (the reference's tools/ctd_train/main.cpp as a library).
//
// Same run semantics as the reference: config keys and defaults, the
// int32-token / int8-mask document format, mt19937_64 document sampling seeded
// with seed + start_step, loss / accum scaling per micro-batch (micro-batches
// with an all-zero mask are skipped), warmup + cosine LR in float, clipping
// over decay-then-no-decay parameters, loss.jsonl records, validation,
// periodic and final checkpoints with the optimizer state, and resume.
// Differences: resume loads offloaded m/v straight into pinned host memory
// (the reference copied device-to-device into them, main.cpp:236-243), and
// the offloaded optimizer streams parameters in model order so the next
// forward overlaps it.
#include "ctd/train.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <fstream>
#include <iostream>
#include <random>
#include <sstream>
#include <stdexcept>

#include "ctd/autograd.h"
#include "ctd/ops/repeat_kv.h"
#include "ctd/runtime.h"
#include "ctd/safetensors.h"
#include "json.h"

namespace ctd::train {

namespace fs = std::filesystem;

namespace {

std::string read_text(const fs::path& p) {
  std::ifstream f(p, std::ios::binary);
  if (!f) throw std::runtime_error("cannot open config " + p.string());
  std::stringstream ss;
  ss << f.rdbuf();
  return ss.str();
}

// Reads a whole data file into `out`, whose element size the file's length
// must be a multiple of.
template <typename T>
void read_array(const fs::path& p, std::vector<T>& out) {
  std::error_code ec;
  const uintmax_t bytes = fs::file_size(p, ec);
  if (ec) throw std::runtime_error("data: cannot stat " + p.string() + " (" + ec.message() + ")");
  if (bytes % sizeof(T) != 0)
    throw std::runtime_error("data: " + p.string() + " is " + std::to_string(bytes) +
                             " bytes, not a whole number of " + std::to_string(sizeof(T)) +
                             "-byte values");
  out.resize(static_cast<size_t>(bytes / sizeof(T)));
  std::ifstream f(p, std::ios::binary);
  if (!f || (bytes > 0 && !f.read(reinterpret_cast<char*>(out.data()),
                                  static_cast<std::streamsize>(bytes))))
    throw std::runtime_error("data: cannot read " + p.string());
}

const json::JVal* key(const json::JVal& j, const char* k) { return j.find(k); }

int get_int(const json::JVal& j, const char* k, int def) {
  const json::JVal* v = key(j, k);
  if (!v) return def;
  if (v->kind != json::JVal::kNum) throw std::runtime_error(std::string("config: ") + k + " must be a number");
  return static_cast<int>(v->num);
}
float get_float(const json::JVal& j, const char* k, float def) {
  const json::JVal* v = key(j, k);
  if (!v) return def;
  if (v->kind != json::JVal::kNum) throw std::runtime_error(std::string("config: ") + k + " must be a number");
  return static_cast<float>(v->num);
}
bool get_bool(const json::JVal& j, const char* k, bool def) {
  const json::JVal* v = key(j, k);
  if (!v) return def;
  if (v->kind != json::JVal::kBool) throw std::runtime_error(std::string("config: ") + k + " must be true/false");
  return v->num != 0;
}
std::string get_string(const json::JVal& j, const char* k) {
  const json::JVal& v = j.at(k);
  if (v.kind != json::JVal::kStr) throw std::runtime_error(std::string("config: ") + k + " must be a string");
  return v.str;
}

// LlamaConfig from a JSON object with the HF config field names.
nn::LlamaConfig model_config(const json::JVal& m) {
  if (m.kind != json::JVal::kObj) throw std::runtime_error("config: model must be an object");
  nn::LlamaConfig a{};
  a.vocab_size = get_int(m, "vocab_size", 0);
  a.hidden_size = get_int(m, "hidden_size", 0);
  a.intermediate_size = get_int(m, "intermediate_size", 0);
  a.num_hidden_layers = get_int(m, "num_hidden_layers", 0);
  a.num_attention_heads = get_int(m, "num_attention_heads", 0);
  a.num_key_value_heads = get_int(m, "num_key_value_heads", a.num_attention_heads);
  a.head_dim = get_int(m, "head_dim",
                       a.num_attention_heads ? a.hidden_size / a.num_attention_heads : 0);
  a.max_position_embeddings = get_int(m, "max_position_embeddings", 8192);
  a.rms_norm_eps = get_float(m, "rms_norm_eps", 1e-5f);
  a.rope_theta = get_float(m, "rope_theta", 1e4f);
  a.tie_word_embeddings = get_bool(m, "tie_word_embeddings", true);
  a.qk_norm = get_bool(m, "qk_norm", false);
  a.rope_scaling_factor = get_float(m, "rope_scaling_factor", 0.0f);
  a.rope_scaling_low_freq_factor = get_float(m, "rope_scaling_low_freq_factor", 1.0f);
  a.rope_scaling_high_freq_factor = get_float(m, "rope_scaling_high_freq_factor", 4.0f);
  a.rope_scaling_original_max_pos = get_int(m, "rope_scaling_original_max_pos", 8192);
  if (a.vocab_size <= 0 || a.hidden_size <= 0 || a.num_hidden_layers <= 0 ||
      a.num_attention_heads <= 0 || a.intermediate_size <= 0)
    throw std::runtime_error("config: model needs vocab_size, hidden_size, intermediate_size, "
                             "num_hidden_layers and num_attention_heads");
  return a;
}

}  // namespace

nn::LlamaConfig load_model_config(const fs::path& path) {
  const std::string text = read_text(path);
  return model_config(json::Parser(text, "model config: bad JSON").parse());
}

Config load_config(const fs::path& cfg_path) {
  const std::string text = read_text(cfg_path);
  const json::JVal j = json::Parser(text, "config: bad JSON").parse();
  if (j.kind != json::JVal::kObj) throw std::runtime_error("config: not a JSON object");
  Config c;
  c.run_dir = cfg_path.parent_path();
  c.run_name = key(j, "run_name") ? get_string(j, "run_name") : c.run_dir.filename().string();
  c.init_weights = get_string(j, "init_weights");
  if (key(j, "resume_from")) c.resume_from = get_string(j, "resume_from");
  c.data_dir = get_string(j, "data_dir");
  c.seq_len = get_int(j, "seq_len", c.seq_len);
  c.batch_size = get_int(j, "batch_size", c.batch_size);
  c.grad_accum_steps = get_int(j, "grad_accum_steps", c.grad_accum_steps);
  c.total_steps = get_int(j, "total_steps", c.total_steps);
  c.warmup_steps = get_int(j, "warmup_steps", c.warmup_steps);
  c.lr = get_float(j, "lr", c.lr);
  c.min_lr_ratio = get_float(j, "min_lr_ratio", c.min_lr_ratio);
  c.weight_decay = get_float(j, "weight_decay", c.weight_decay);
  c.beta1 = get_float(j, "beta1", c.beta1);
  c.beta2 = get_float(j, "beta2", c.beta2);
  c.eps = get_float(j, "eps", c.eps);
  c.clip_grad_norm = get_float(j, "clip_grad_norm", c.clip_grad_norm);
  c.val_every = get_int(j, "val_every", c.val_every);
  c.save_every = get_int(j, "save_every", c.save_every);
  c.log_every = get_int(j, "log_every", c.log_every);
  if (const json::JVal* s = key(j, "seed")) {
    if (s->kind != json::JVal::kNum) throw std::runtime_error("config: seed must be a number");
    c.seed = std::stoull(s->str);
  }
  c.offload_optimizer = get_bool(j, "offload_optimizer", c.offload_optimizer);
  c.gradient_checkpointing = get_bool(j, "gradient_checkpointing", c.gradient_checkpointing);
  if (const json::JVal* m = key(j, "model")) {
    c.model = model_config(*m);
    c.has_model = true;
  }
  if (c.seq_len < 2 || c.batch_size < 1 || c.grad_accum_steps < 1)
    throw std::runtime_error("config: seq_len >= 2, batch_size >= 1 and grad_accum_steps >= 1");
  return c;
}

DataSplit load_split(const fs::path& tok_path, const fs::path& mask_path, int seq_len) {
  if (seq_len < 2) throw std::runtime_error("load_split: seq_len must be >= 2");
  DataSplit s;
  read_array(tok_path, s.tokens);
  read_array(mask_path, s.masks);
  const size_t per_doc = static_cast<size_t>(seq_len);
  if (s.tokens.size() % per_doc != 0)
    throw std::runtime_error("data: " + tok_path.string() + " holds " +
                             std::to_string(s.tokens.size()) + " tokens, not whole documents of " +
                             std::to_string(seq_len));
  s.num_docs = static_cast<int64_t>(s.tokens.size() / per_doc);
  if (s.masks.size() != s.tokens.size())
    throw std::runtime_error("data: " + mask_path.string() + " has " +
                             std::to_string(s.masks.size()) + " mask values for " +
                             std::to_string(s.tokens.size()) + " tokens");
  return s;
}

HostBatch make_host_batch(const DataSplit& split, const std::vector<int64_t>& doc_indices,
                          int seq_len) {
  HostBatch h;
  h.B = static_cast<int64_t>(doc_indices.size());
  h.T = seq_len - 1;
  const size_t n = static_cast<size_t>(h.B * h.T);
  h.input_ids.resize(n);
  h.targets.resize(n);
  h.loss_mask.resize(n);
  for (int64_t b = 0; b < h.B; ++b) {
    const int64_t doc = doc_indices[static_cast<size_t>(b)];
    if (doc < 0 || doc >= split.num_docs) throw std::runtime_error("make_batch: document index out of range");
    const int32_t* tok = split.tokens.data() + doc * seq_len;
    const int8_t* msk = split.masks.data() + doc * seq_len;
    for (int64_t t = 0; t < h.T; ++t) {
      const size_t i = static_cast<size_t>(b * h.T + t);
      h.input_ids[i] = tok[t];
      h.targets[i] = tok[t + 1];
      const float m = static_cast<float>(msk[t + 1]);
      h.loss_mask[i] = m;
      h.sum_mask += m;  // float accumulation in document order, as the reference
    }
  }
  return h;
}

Batch make_batch(const DataSplit& split, const std::vector<int64_t>& doc_indices, int seq_len,
                 Device device) {
  const HostBatch h = make_host_batch(split, doc_indices, seq_len);
  const std::vector<int64_t> shape = {h.B, h.T};
  Batch out;
  out.input_ids = Tensor::from_host(h.input_ids.data(), shape, DType::kInt64, device);
  out.targets = Tensor::from_host(h.targets.data(), shape, DType::kInt64, device);
  out.loss_mask = Tensor::from_host(h.loss_mask.data(), shape, DType::kFloat32, device);
  out.sum_mask = h.sum_mask;
  return out;
}

float lr_at_step(int step, const Config& c) {
  if (step < c.warmup_steps) {
    const float t = static_cast<float>(step) / static_cast<float>(std::max(1, c.warmup_steps));
    return c.lr * t;
  }
  const int decay_steps = std::max(1, c.total_steps - c.warmup_steps);
  const int s = std::min(step - c.warmup_steps, decay_steps);
  const float t = static_cast<float>(s) / static_cast<float>(decay_steps);
  const float cos_factor = 0.5f * (1.0f + std::cos(static_cast<float>(M_PI) * t));
  const float min_lr = c.lr * c.min_lr_ratio;
  return min_lr + (c.lr - min_lr) * cos_factor;
}

float run_val(const nn::Model& model, const DataSplit& val, int seq_len, Device device) {
  // Documents go to the device in groups of about kValGroupTokens tokens (one
  // batch of copies each); each document is then one forward over row views
  // of its group, its loss left on the device until the group's forwards are
  // queued, so a group has one round trip and the device holds one group's
  // inputs at a time however large the split.  Weighting and skipping follow
  // main.cpp:195-207: each document's masked-mean loss weighs by its own mask
  // sum (summed in float, in token order, like make_host_batch), documents
  // without targets are skipped, and the weighted sum is formed in double in
  // document order.
  constexpr int64_t kValGroupTokens = int64_t{1} << 20;
  if (val.num_docs == 0) return 0.0f;
  const int64_t per_group = std::max<int64_t>(1, kValGroupTokens / std::max(seq_len, 1));
  autograd::NoGradGuard no_grad;
  double num = 0.0, den = 0.0;
  for (int64_t d0 = 0; d0 < val.num_docs; d0 += per_group) {
    const int64_t d1 = std::min(val.num_docs, d0 + per_group);
    std::vector<int64_t> docs(static_cast<size_t>(d1 - d0));
    for (int64_t i = d0; i < d1; ++i) docs[static_cast<size_t>(i - d0)] = i;
    const HostBatch h = make_host_batch(val, docs, seq_len);
    const int64_t T = h.T;
    const Tensor ids = Tensor::from_host(h.input_ids.data(), {h.B, T}, DType::kInt64, device);
    const Tensor tgt = Tensor::from_host(h.targets.data(), {h.B, T}, DType::kInt64, device);
    const Tensor msk = Tensor::from_host(h.loss_mask.data(), {h.B, T}, DType::kFloat32, device);
    std::vector<float> weight;
    std::vector<Tensor> losses;
    for (int64_t d = 0; d < h.B; ++d) {
      float w = 0.0f;
      for (int64_t t = 0; t < T; ++t) w += h.loss_mask[static_cast<size_t>(d * T + t)];
      if (w <= 0.0f) continue;
      losses.push_back(model.forward_train_masked(ids.view_at(d * T, {1, T}),
                                                  tgt.view_at(d * T, {1, T}),
                                                  msk.view_at(d * T, {1, T})));
      weight.push_back(w);
    }
    for (size_t i = 0; i < losses.size(); ++i) {
      float l = 0.0f;
      losses[i].copy_to_host(&l);
      num += static_cast<double>(l) * static_cast<double>(weight[i]);
      den += static_cast<double>(weight[i]);
    }
  }
  return den > 0.0 ? static_cast<float>(num / den) : 0.0f;
}

fs::path opt_path_for(const fs::path& weights_path) {
  return weights_path.string() + ".opt.safetensors";
}

void save_optimizer_state(optim::AdamW& opt, const nn::Model::NamedParameters& named,
                          const fs::path& path) {
  std::vector<std::pair<std::string, Tensor>> items;
  items.reserve(2 * named.all.size() + 1);
  for (size_t i = 0; i < named.decay_names.size(); ++i) {
    items.emplace_back("optimizer.m." + named.decay_names[i], opt.m_tensor(0, i));
    items.emplace_back("optimizer.v." + named.decay_names[i], opt.v_tensor(0, i));
  }
  for (size_t i = 0; i < named.no_decay_names.size(); ++i) {
    items.emplace_back("optimizer.m." + named.no_decay_names[i], opt.m_tensor(1, i));
    items.emplace_back("optimizer.v." + named.no_decay_names[i], opt.v_tensor(1, i));
  }
  runtime::synchronize();
  const float step_f = static_cast<float>(opt.step_count());
  items.emplace_back("optimizer.step", Tensor::from_host(&step_f, {1}, DType::kFloat32, kCPU));
  save_safetensors(items, path);
}

void load_optimizer_state(optim::AdamW& opt, const nn::Model::NamedParameters& named,
                          const fs::path& path) {
  // Each m/v entry is read straight into the optimizer's own buffer: pinned
  // host memory when offloaded, device memory otherwise.
  const SafetensorsReader file(path);
  opt.ensure_state_initialized();
  const std::vector<std::string>* names[2] = {&named.decay_names, &named.no_decay_names};
  for (int g = 0; g < 2; ++g)
    for (size_t i = 0; i < names[g]->size(); ++i) {
      const std::string& n = (*names[g])[i];
      for (const char* which : {"m", "v"}) {
        const std::string k = std::string("optimizer.") + which + "." + n;
        if (!file.find(k)) throw std::runtime_error("resume: " + path.string() + " lacks " + k);
        Tensor dst = which[0] == 'm' ? opt.m_tensor(g, i) : opt.v_tensor(g, i);
        file.read(k, dst);
      }
    }
  Tensor step = Tensor::empty({1}, DType::kFloat32, kCPU);
  if (!file.find("optimizer.step"))
    throw std::runtime_error("resume: " + path.string() + " lacks optimizer.step");
  file.read("optimizer.step", step);
  opt.set_step_count(static_cast<int64_t>(*static_cast<const float*>(step.data_ptr())));
}

std::string train_event(int step, float loss, float lr, float grad_norm, double tokens_per_sec,
                        double wall_s) {
  return json::ObjectWriter()
      .field("grad_norm", grad_norm)
      .field("loss", loss)
      .field("lr", lr)
      .field("phase", "train")
      .field("step", step)
      .field("tokens_per_sec", tokens_per_sec)
      .field("wall_s", wall_s)
      .str();
}

std::string val_event(int step, float loss, double wall_s) {
  return json::ObjectWriter()
      .field("loss", loss)
      .field("phase", "val")
      .field("step", step)
      .field("wall_s", wall_s)
      .str();
}

int run(const Config& cfg) {
  using clock = std::chrono::steady_clock;
  fs::create_directories(cfg.run_dir);
  std::cerr << "ctd_train: run " << cfg.run_name << " in " << cfg.run_dir << "\n";
  const bool resuming = !cfg.resume_from.empty();
  const fs::path weights_path = resuming ? cfg.resume_from : cfg.init_weights;
  std::cerr << "ctd_train: " << (resuming ? "resume weights " : "initial weights ")
            << weights_path << "\n";
  TensorDict weights = load_safetensors(weights_path, kHIP0);
  const nn::LlamaConfig arch = cfg.has_model ? cfg.model : nn::autodetect_config(weights);
  nn::Model model = nn::build_model(weights, arch);
  weights.clear();
  model.gradient_checkpointing = cfg.gradient_checkpointing;
  auto named = model.collect_parameters();
  std::cerr << "ctd_train: " << named.all.size() << " parameter tensors (" << named.decay.size()
            << " with weight decay)\n";

  std::vector<Tensor> all_params;
  all_params.insert(all_params.end(), named.decay.begin(), named.decay.end());
  all_params.insert(all_params.end(), named.no_decay.begin(), named.no_decay.end());

  std::vector<optim::ParamGroup> groups = {{named.decay, cfg.lr, cfg.weight_decay},
                                           {named.no_decay, cfg.lr, 0.0f}};
  optim::AdamW opt(std::move(groups), cfg.beta1, cfg.beta2, cfg.eps, cfg.offload_optimizer);
  if (cfg.offload_optimizer) {
    // Model order (collect_parameters), mapped onto the two groups.
    std::vector<std::pair<size_t, size_t>> order;
    size_t di = 0, ni = 0;
    for (const auto& [name, p] : named.all) {
      (void)p;
      if (di < named.decay_names.size() && named.decay_names[di] == name)
        order.emplace_back(0, di++);
      else
        order.emplace_back(1, ni++);
    }
    opt.set_update_order(std::move(order));
  }
  // The last micro-batch's backward stages the first parameters' optimizer
  // state while the host link is idle; clearing the hook on the way out keeps
  // the model from calling into the optimizer after it is gone.
  bool prefetch_armed = false;
  struct HookReset {
    nn::Model& m;
    ~HookReset() { m.recompute_hook = nullptr; }
  } hook_reset{model};
  if (cfg.offload_optimizer) {
    const int at = optimizer_prefetch_layer(
        model.config, static_cast<int64_t>(cfg.batch_size) * cfg.seq_len);
    model.recompute_hook = [&opt, &prefetch_armed, at](int layer) {
      if (prefetch_armed && layer == at) opt.prefetch();
    };
  }

  int64_t start_step = 0;
  if (resuming) {
    const fs::path op = opt_path_for(cfg.resume_from);
    if (fs::exists(op)) {
      load_optimizer_state(opt, named, op);
      start_step = opt.step_count();
      std::cerr << "ctd_train: optimizer state from " << op << ", next step " << start_step + 1
                << "\n";
    } else {
      std::cerr << "ctd_train: " << op << " not found: m and v start from zero and the "
                << "schedule from step 1\n";
    }
  }

  const DataSplit train = load_split(cfg.data_dir / "train.bin", cfg.data_dir / "train_mask.bin",
                                     cfg.seq_len);
  const DataSplit val = load_split(cfg.data_dir / "val.bin", cfg.data_dir / "val_mask.bin",
                                   cfg.seq_len);
  if (train.num_docs < 1) throw std::runtime_error("train split is empty");
  std::cerr << "ctd_train: " << train.num_docs << " training and " << val.num_docs
            << " validation documents\n";

  std::mt19937_64 rng(cfg.seed + static_cast<uint64_t>(start_step));
  std::uniform_int_distribution<int64_t> pick(0, train.num_docs - 1);

  const fs::path log_path = cfg.run_dir / "loss.jsonl";
  std::ofstream log(log_path, resuming ? (std::ios::out | std::ios::app)
                                       : (std::ios::out | std::ios::trunc));
  if (!log) throw std::runtime_error("cannot open log " + log_path.string());

  const auto t_run_start = clock::now();
  const float inv_accum = 1.0f / static_cast<float>(cfg.grad_accum_steps);
  for (int step = static_cast<int>(start_step) + 1; step <= cfg.total_steps; ++step) {
    const auto t_step_start = clock::now();
    double accum_loss = 0.0, accum_active = 0.0;
    for (int micro = 0; micro < cfg.grad_accum_steps; ++micro) {
      std::vector<int64_t> idx(static_cast<size_t>(cfg.batch_size));
      for (auto& i : idx) i = pick(rng);
      Batch b = make_batch(train, idx, cfg.seq_len, kHIP0);
      if (b.sum_mask <= 0.0f) continue;
      Tensor loss = model.forward_train_masked(b.input_ids, b.targets, b.loss_mask);
      Tensor scaled = ops::mul_scalar(loss, inv_accum);
      prefetch_armed = micro == cfg.grad_accum_steps - 1;
      scaled.backward();
      prefetch_armed = false;
      float l = 0.0f;
      loss.copy_to_host(&l);
      accum_loss += static_cast<double>(l) * static_cast<double>(b.sum_mask);
      accum_active += static_cast<double>(b.sum_mask);
    }
    const float lr = lr_at_step(step, cfg);
    opt.set_lr(lr);
    const float grad_norm = optim::clip_grad_norm_(all_params, cfg.clip_grad_norm);
    opt.step();
    opt.zero_grad();

    const auto t_step_end = clock::now();
    const double step_s = std::chrono::duration<double>(t_step_end - t_step_start).count();
    const double wall_s = std::chrono::duration<double>(t_step_end - t_run_start).count();
    const double tps = accum_active / std::max(step_s, 1e-9);
    const float train_loss =
        accum_active > 0.0 ? static_cast<float>(accum_loss / accum_active) : 0.0f;
    if (cfg.log_every > 0 && step % cfg.log_every == 0) {
      log << train_event(step, train_loss, lr, grad_norm, tps, wall_s) << "\n";
      log.flush();
      std::cerr << "ctd_train: step " << step << " of " << cfg.total_steps << "  loss "
                << train_loss << "  lr " << lr << "  grad norm " << grad_norm << "  "
                << static_cast<int64_t>(tps) << " tokens/s\n";
    }
    if (cfg.val_every > 0 && step % cfg.val_every == 0) {
      const float vl = run_val(model, val, cfg.seq_len, kHIP0);
      const double w = std::chrono::duration<double>(clock::now() - t_run_start).count();
      log << val_event(step, vl, w) << "\n";
      log.flush();
      std::cerr << "ctd_train: step " << step << "  validation loss " << vl << "\n";
    }
    if (cfg.save_every > 0 && step % cfg.save_every == 0) {
      const fs::path ckpt = cfg.run_dir / ("ckpt_step_" + std::to_string(step) + ".safetensors");
      runtime::synchronize();
      save_safetensors(named.all, ckpt);
      save_optimizer_state(opt, named, opt_path_for(ckpt));
      std::cerr << "ctd_train: step " << step << "  wrote " << ckpt << " and its optimizer state\n";
    }
  }
  const fs::path final_ckpt = cfg.run_dir / "final.safetensors";
  runtime::synchronize();
  save_safetensors(named.all, final_ckpt);
  save_optimizer_state(opt, named, opt_path_for(final_ckpt));
  std::cerr << "ctd_train: finished; wrote " << final_ckpt << " and its optimizer state\n";
  return 0;
}

}  // namespace ctd::train
