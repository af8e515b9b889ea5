// C entry points (include/ctd_capi.h) over the C++ layer: model construction
// with seeded synthetic weights, the ctd_train step, memory statistics and
// checkpoint save/load.  The step follows tools/ctd_train/main.cpp:348-398 of
// the reference (forward_train_masked, backward, clip_grad_norm_, step,
// zero_grad); the optimizer-state file follows main.cpp:208-271 (m then v per
// parameter, decay group first, plus optimizer.step), loading straight into
// the pinned host state when m/v are offloaded.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "ctd/ops/attention.h"
#include "ctd/allocator.h"
#include "ctd/generate.h"
#include "ctd/nn/model.h"
#include "ctd/ops/loss.h"
#include "ctd/ops/repeat_kv.h"
#include "ctd/optim.h"
#include "ctd/runtime.h"
#include "ctd/sampling.h"
#include "ctd/train.h"
#include "ctd_capi.h"
#include "block_arena.h"

using namespace ctd;

namespace {

thread_local std::string g_last_error;

template <typename F>
int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_last_error = e.what();
  } catch (...) {
    g_last_error = "unknown C++ exception";
  }
  return CTD_EXCEPTION;
}

uint64_t splitmix(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

nn::LlamaConfig to_llama(const ctd_model_config& c) {
  nn::LlamaConfig l{};
  l.vocab_size = c.vocab_size;
  l.hidden_size = c.hidden_size;
  l.intermediate_size = c.intermediate_size;
  l.num_hidden_layers = c.num_layers;
  l.num_attention_heads = c.num_heads;
  l.num_key_value_heads = c.num_kv_heads;
  l.head_dim = c.head_dim;
  l.max_position_embeddings = 1 << 20;
  l.rms_norm_eps = c.rms_norm_eps;
  l.rope_theta = c.rope_theta;
  l.tie_word_embeddings = true;
  l.qk_norm = c.qk_norm != 0;
  l.rope_scaling_factor = c.rope_factor;
  l.rope_scaling_low_freq_factor = c.rope_low_freq_factor;
  l.rope_scaling_high_freq_factor = c.rope_high_freq_factor;
  l.rope_scaling_original_max_pos = c.rope_original_max_pos;
  return l;
}

ctd_model_config from_llama(const nn::LlamaConfig& l) {
  ctd_model_config c{};
  c.vocab_size = l.vocab_size;
  c.hidden_size = l.hidden_size;
  c.intermediate_size = l.intermediate_size;
  c.num_layers = l.num_hidden_layers;
  c.num_heads = l.num_attention_heads;
  c.num_kv_heads = l.num_key_value_heads;
  c.head_dim = l.head_dim;
  c.qk_norm = l.qk_norm ? 1 : 0;
  c.rms_norm_eps = l.rms_norm_eps;
  c.rope_theta = l.rope_theta;
  c.rope_factor = l.rope_scaling_factor;
  c.rope_low_freq_factor = l.rope_scaling_low_freq_factor;
  c.rope_high_freq_factor = l.rope_scaling_high_freq_factor;
  c.rope_original_max_pos = l.rope_scaling_original_max_pos;
  return c;
}

struct Trainer {
  nn::Model model;
  nn::Model::NamedParameters named;
  std::vector<int32_t> decay;  // per entry of named.all
  std::vector<std::pair<size_t, size_t>> opt_index;  // named.all index -> (group, position)
  Tensor ids, targets, mask;
  int64_t B = 0, T = 0;
  float mask_sum = 0.f;
  std::unique_ptr<optim::AdamW> opt;
  // Set while train_step's backward runs: only then does the model's
  // recompute hook start the offloaded optimizer's prefetch.
  bool prefetch_armed = false;
  // Layer whose re-run starts it: >= 0 that layer, -1 never, -2 the estimate
  // of train::optimizer_prefetch_layer for the batch.
  int prefetch_layer = -2;
};


// Decay group, then no-decay group: the order ctd_train hands the parameters
// to clip_grad_norm_ (tools/ctd_train/main.cpp:296-299), which fixes the order
// of the norm's reduction.
std::vector<Tensor> clip_order(const Trainer& tr) {
  std::vector<Tensor> ps(tr.named.decay.begin(), tr.named.decay.end());
  ps.insert(ps.end(), tr.named.no_decay.begin(), tr.named.no_decay.end());
  return ps;
}

Trainer* as_trainer(ctd_trainer_t t) {
  if (!t) throw std::runtime_error("null trainer handle");
  return static_cast<Trainer*>(t);
}

Tensor& param_at(Trainer* tr, int64_t i) {
  if (i < 0 || i >= static_cast<int64_t>(tr->named.all.size()))
    throw std::runtime_error("parameter index out of range");
  return tr->named.all[static_cast<size_t>(i)].second;
}

void check_numel(const Tensor& t, int64_t numel) {
  if (t.numel() != numel) throw std::runtime_error("numel mismatch");
}

// Uninitialised device tensors under the HF names build_model expects.
TensorDict weight_shapes(const nn::LlamaConfig& c) {
  TensorDict w;
  const int64_t d = c.hidden_size, I = c.intermediate_size, H = c.num_attention_heads,
                Hk = c.num_key_value_heads, D = c.head_dim, V = c.vocab_size;
  auto mk = [&](const std::string& name, std::vector<int64_t> shape) {
    w.emplace(name, Tensor::empty(std::move(shape), DType::kFloat32, kHIP0));
  };
  mk("model.embed_tokens.weight", {V, d});
  mk("model.norm.weight", {d});
  for (int l = 0; l < c.num_hidden_layers; ++l) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    mk(p + "input_layernorm.weight", {d});
    mk(p + "post_attention_layernorm.weight", {d});
    mk(p + "self_attn.q_proj.weight", {H * D, d});
    mk(p + "self_attn.k_proj.weight", {Hk * D, d});
    mk(p + "self_attn.v_proj.weight", {Hk * D, d});
    mk(p + "self_attn.o_proj.weight", {d, H * D});
    if (c.qk_norm) {
      mk(p + "self_attn.q_norm.weight", {D});
      mk(p + "self_attn.k_norm.weight", {D});
    }
    mk(p + "mlp.gate_proj.weight", {I, d});
    mk(p + "mlp.up_proj.weight", {I, d});
    mk(p + "mlp.down_proj.weight", {d, I});
  }
  return w;
}

}  // namespace

extern "C" {

const char* ctd_last_error(void) { return g_last_error.c_str(); }

int ctd_preset_config(const char* name, ctd_model_config* out) {
  return guarded([&] {
    if (!name || !out) throw std::runtime_error("null argument");
    const std::string n(name);
    nn::LlamaConfig l;
    if (n == "smollm2-135m") l = nn::smollm2_135m_config();
    else if (n == "smollm2-360m") l = nn::smollm2_360m_config();
    else if (n == "qwen3-0.6b") l = nn::qwen3_0_6b_config();
    else if (n == "qwen3-1.7b") l = nn::qwen3_1_7b_config();
    else if (n == "llama3.2-1b") l = nn::llama3_2_1b_config();
    else throw std::runtime_error("unknown preset " + n);
    *out = from_llama(l);
  });
}

int ctd_trainer_create(const ctd_model_config* cfg, uint64_t seed, float init_std,
                       float norm_value, ctd_trainer_t* out) {
  return guarded([&] {
    if (!cfg || !out) throw std::runtime_error("null argument");
    auto tr = std::make_unique<Trainer>();
    const nn::LlamaConfig l = to_llama(*cfg);
    TensorDict w = weight_shapes(l);
    tr->model = nn::build_model(w, l);
    tr->named = tr->model.collect_parameters();
    // Seeded init over the parameter list in collect_parameters order: one
    // counter stream, element offset = running parameter offset.
    uint64_t offset = 0;
    size_t di = 0, ni = 0;
    for (auto& [name, p] : tr->named.all) {
      const bool is_norm = p.dim() == 1;
      const bool dec = di < tr->named.decay_names.size() && tr->named.decay_names[di] == name;
      if (dec) {
        tr->opt_index.emplace_back(0, di++);
      } else {
        tr->opt_index.emplace_back(1, ni++);
      }
      tr->decay.push_back(dec ? 1 : 0);
      if (is_norm && !std::isnan(norm_value)) {
        CTD_CHECK(ember_fill(static_cast<float*>(p.data_ptr()), p.numel(), norm_value,
                             runtime::compute_stream()));
      } else {
        CTD_CHECK(ember_fill_normal(static_cast<float*>(p.data_ptr()), p.numel(), seed, offset,
                                    0.0f, init_std, runtime::compute_stream()));
      }
      offset += static_cast<uint64_t>(p.numel());
    }
    runtime::synchronize();
    *out = tr.release();
  });
}

int ctd_trainer_destroy(ctd_trainer_t t) {
  return guarded([&] {
    runtime::synchronize();
    delete static_cast<Trainer*>(t);
  });
}

int ctd_trainer_num_params(ctd_trainer_t t, int64_t* n) {
  return guarded([&] { *n = static_cast<int64_t>(as_trainer(t)->named.all.size()); });
}

int ctd_trainer_param_info(ctd_trainer_t t, int64_t i, char* name, size_t cap, int64_t* numel,
                           int32_t* decay) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    Tensor& p = param_at(tr, i);
    const std::string& nm = tr->named.all[static_cast<size_t>(i)].first;
    if (name && cap) {
      std::strncpy(name, nm.c_str(), cap - 1);
      name[cap - 1] = '\0';
    }
    if (numel) *numel = p.numel();
    if (decay) *decay = tr->decay[static_cast<size_t>(i)];
  });
}

int ctd_trainer_set_param(ctd_trainer_t t, int64_t i, const float* host, int64_t numel) {
  return guarded([&] {
    Tensor& p = param_at(as_trainer(t), i);
    check_numel(p, numel);
    CTD_CHECK(ember_memcpy_async(p.data_ptr(), host, p.nbytes(), 0, runtime::compute_stream()));
    runtime::synchronize();
  });
}

int ctd_trainer_get_param(ctd_trainer_t t, int64_t i, float* host, int64_t numel) {
  return guarded([&] {
    Tensor& p = param_at(as_trainer(t), i);
    check_numel(p, numel);
    p.copy_to_host(host);
  });
}

int ctd_trainer_get_grad(ctd_trainer_t t, int64_t i, float* host, int64_t numel) {
  try {
    Tensor g = param_at(as_trainer(t), i).grad();
    if (!g.storage()) return -1;
    check_numel(g, numel);
    g.copy_to_host(host);
    return 0;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return CTD_EXCEPTION;
  }
}

int ctd_trainer_set_checkpointing(ctd_trainer_t t, int32_t on) {
  return guarded([&] { as_trainer(t)->model.gradient_checkpointing = on != 0; });
}

int ctd_trainer_set_batch(ctd_trainer_t t, const int64_t* ids, const int64_t* targets,
                          const float* mask, int64_t B, int64_t T) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (B <= 0 || T <= 0 || !ids || !targets) throw std::runtime_error("bad batch");
    std::vector<float> ones;
    if (!mask) {
      ones.assign(static_cast<size_t>(B * T), 1.0f);
      mask = ones.data();
    }
    double ms = 0.0;
    for (int64_t i = 0; i < B * T; ++i) ms += mask[i];
    tr->ids = Tensor::from_host(ids, {B, T}, DType::kInt64, kHIP0);
    tr->targets = Tensor::from_host(targets, {B, T}, DType::kInt64, kHIP0);
    tr->mask = Tensor::from_host(mask, {B, T}, DType::kFloat32, kHIP0);
    tr->B = B;
    tr->T = T;
    tr->mask_sum = static_cast<float>(ms);
  });
}

int ctd_trainer_synthetic_batch(ctd_trainer_t t, int64_t B, int64_t T, uint64_t seed,
                                int32_t masked) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    const uint64_t V = static_cast<uint64_t>(tr->model.config.vocab_size);
    uint64_t s = seed * 0x2545F4914F6CDD1Dull + 1;
    std::vector<int64_t> ids(static_cast<size_t>(B * T)), tg(static_cast<size_t>(B * T));
    std::vector<float> mask(static_cast<size_t>(B * T), 1.0f);
    for (int64_t b = 0; b < B; ++b) {
      std::vector<int64_t> row(static_cast<size_t>(T + 1));
      for (auto& x : row) x = static_cast<int64_t>(splitmix(s) % V);
      for (int64_t i = 0; i < T; ++i) {
        ids[static_cast<size_t>(b * T + i)] = row[static_cast<size_t>(i)];
        tg[static_cast<size_t>(b * T + i)] = row[static_cast<size_t>(i + 1)];
      }
      if (masked) {
        const double u = 0.2 + 0.4 * (static_cast<double>(splitmix(s) >> 11) / 9007199254740992.0);
        const int64_t cut = static_cast<int64_t>(std::floor(u * static_cast<double>(T)));
        for (int64_t i = 0; i < cut; ++i) mask[static_cast<size_t>(b * T + i)] = 0.0f;
      }
    }
    if (ctd_trainer_set_batch(t, ids.data(), tg.data(), mask.data(), B, T) != 0)
      throw std::runtime_error(g_last_error);
  });
}

int ctd_trainer_forward_backward(ctd_trainer_t t, int32_t backward, float* loss) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->ids.defined()) throw std::runtime_error("no batch set");
    Tensor l = tr->model.forward_train_masked(tr->ids, tr->targets, tr->mask);
    if (backward) l.backward();
    if (loss) l.copy_to_host(loss);
  });
}

int ctd_trainer_hidden(ctd_trainer_t t, float* host, int64_t numel) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    autograd::NoGradGuard ng;
    Tensor h = tr->model.embed_tokens.forward(tr->ids);
    for (const auto& layer : tr->model.layers) h = layer.forward_train(h);
    h = tr->model.norm.forward(h);
    check_numel(h, numel);
    h.copy_to_host(host);
  });
}

int ctd_trainer_block_step(ctd_trainer_t t, int64_t layer, const float* x, const float* dy,
                           int64_t B, int64_t T, int32_t checkpoint, float* y_out, float* dx_out) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (layer < 0 || layer >= static_cast<int64_t>(tr->model.layers.size()))
      throw std::runtime_error("layer index out of range");
    const auto& blk = tr->model.layers[static_cast<size_t>(layer)];
    const int64_t d = tr->model.config.hidden_size;
    Tensor xin = Tensor::from_host(x, {B, T, d}, DType::kFloat32, kHIP0);
    xin.requires_grad_(true);
    // The checkpoint's re-run in the backward pass takes the model's form,
    // which records the block output's graph without computing it.
    auto fn = [&blk](const Tensor& v) {
      return autograd::is_grad_enabled() ? blk.forward_train_for_backward(v)
                                         : blk.forward_train(v);
    };
    Tensor y = checkpoint ? autograd::checkpoint(fn, xin) : blk.forward_train(xin);
    if (y_out) y.copy_to_host(y_out);
    Tensor g = Tensor::from_host(dy, {B, T, d}, DType::kFloat32, kHIP0);
    y.backward(g);
    if (dx_out) {
      Tensor dx = xin.grad();
      if (!dx.storage()) throw std::runtime_error("block_step: input received no gradient");
      dx.copy_to_host(dx_out);
    }
  });
}

int ctd_trainer_make_optimizer(ctd_trainer_t t, float lr, float weight_decay, float beta1,
                               float beta2, float eps, int32_t offload, int64_t chunk_elems) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    // Two groups like ctd_train (main.cpp:299-311): decay, then no_decay with wd 0.
    std::vector<optim::ParamGroup> groups{{tr->named.decay, lr, weight_decay},
                                          {tr->named.no_decay, lr, 0.0f}};
    tr->model.recompute_hook = nullptr;
    tr->opt = std::make_unique<optim::AdamW>(std::move(groups), beta1, beta2, eps, offload != 0);
    if (offload) {
      tr->model.recompute_hook = [tr](int layer) {
        if (!tr->prefetch_armed) return;
        const int at = tr->prefetch_layer >= -1
                           ? tr->prefetch_layer
                           : train::optimizer_prefetch_layer(tr->model.config, tr->B * tr->T);
        if (layer == at) tr->opt->prefetch();
      };
    }
    if (chunk_elems > 0) tr->opt->set_offload_chunk(chunk_elems);
    // Stream parameters in model order (collect_parameters), the order in
    // which the forward reads them, so it can overlap the offloaded update.
    tr->opt->set_update_order(tr->opt_index);
    tr->opt->ensure_state_initialized();
  });
}

int ctd_trainer_clip(ctd_trainer_t t, float max_norm, float* total_norm) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    const float v = optim::clip_grad_norm_(clip_order(*tr), max_norm);
    if (total_norm) *total_norm = v;
  });
}

int ctd_trainer_opt_step(ctd_trainer_t t) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->opt) throw std::runtime_error("no optimizer");
    tr->opt->step();
  });
}

int ctd_trainer_zero_grad(ctd_trainer_t t) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    for (auto& [n, p] : tr->named.all) p.zero_grad_();
  });
}

int ctd_trainer_get_opt_state(ctd_trainer_t t, int64_t i, float* m, float* v, int64_t numel) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->opt) throw std::runtime_error("no optimizer");
    param_at(tr, i);
    const auto [gi, pi] = tr->opt_index[static_cast<size_t>(i)];
    runtime::synchronize();
    Tensor& tm = tr->opt->m_tensor(gi, pi);
    Tensor& tv = tr->opt->v_tensor(gi, pi);
    check_numel(tm, numel);
    if (m) tm.copy_to_host(m);
    if (v) tv.copy_to_host(v);
  });
}

int ctd_trainer_offload_stats(ctd_trainer_t t, double* stream_ms, double* bytes_per_direction,
                              double* prefetched_bytes) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    double ms = 0.0, b = 0.0, pf = 0.0;
    if (tr->opt && tr->opt->is_offloaded()) {
      tr->opt->wait_idle();
      const optim::OffloadStats& st = tr->opt->offload_stats();
      ms = st.last_stream_ms;
      b = st.last_d2h_bytes;
      pf = st.last_prefetch_bytes;
    }
    if (stream_ms) *stream_ms = ms;
    if (bytes_per_direction) *bytes_per_direction = b;
    if (prefetched_bytes) *prefetched_bytes = pf;
  });
}

int ctd_trainer_offload_detail(ctd_trainer_t t, ctd_offload_detail* out) {
  return guarded([&] {
    if (!out) throw std::runtime_error("null argument");
    Trainer* tr = as_trainer(t);
    *out = ctd_offload_detail{};
    if (!tr->opt || !tr->opt->is_offloaded()) return;
    tr->opt->wait_idle();
    const optim::OffloadStats& st = tr->opt->offload_stats();
    out->stream_ms = st.last_stream_ms;
    out->h2d_ms = st.last_h2d_ms;
    out->d2h_ms = st.last_d2h_ms;
    out->h2d_bytes = st.last_h2d_bytes;
    out->d2h_bytes = st.last_d2h_bytes;
    out->prefetch_bytes = st.last_prefetch_bytes;
    out->skipped_bytes = st.last_skipped_bytes;
  });
}

int ctd_trainer_set_prefetch_chunks(ctd_trainer_t t, int64_t chunks) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->opt) throw std::runtime_error("no optimizer");
    if (chunks < 0) throw std::runtime_error("prefetch chunks must be >= 0");
    tr->opt->set_prefetch_chunks(chunks);
  });
}

int ctd_trainer_set_prefetch_layer(ctd_trainer_t t, int32_t layer) {
  return guarded([&] {
    if (layer < -2) throw std::runtime_error("prefetch layer must be >= -2");
    as_trainer(t)->prefetch_layer = layer;
  });
}

int ctd_trainer_step_count(ctd_trainer_t t, int64_t* steps) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    *steps = tr->opt ? tr->opt->step_count() : 0;
  });
}

int ctd_trainer_train_step(ctd_trainer_t t, float max_norm, ctd_step_times* times) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->opt) throw std::runtime_error("no optimizer");
    if (!tr->ids.defined()) throw std::runtime_error("no batch set");
    ember_stream_t cs = runtime::compute_stream();
    ember_event_t ev[5];
    for (auto& e : ev) CTD_CHECK(ember_event_create(&e));
    CTD_CHECK(ember_event_record(ev[0], cs));
    mark_allocation_history("forward");
    Tensor loss = tr->model.forward_train_masked(tr->ids, tr->targets, tr->mask);
    CTD_CHECK(ember_event_record(ev[1], cs));
    sample_device_memory();
    mark_allocation_history("backward");
    {
      struct Arm {
        bool& flag;
        ~Arm() { flag = false; }
      } arm{tr->prefetch_armed};
      tr->prefetch_armed = true;
      loss.backward();
    }
    CTD_CHECK(ember_event_record(ev[2], cs));
    sample_device_memory();
    mark_allocation_history("clip+step");
    float gn = 0.f;
    if (max_norm > 0.f) {
      gn = optim::clip_grad_norm_(clip_order(*tr), max_norm);
    }
    CTD_CHECK(ember_event_record(ev[3], cs));
    tr->opt->step();
    CTD_CHECK(ember_event_record(ev[4], cs));
    sample_device_memory();
    for (auto& [n, p] : tr->named.all) p.zero_grad_();
    float lv = 0.f;
    loss.copy_to_host(&lv);
    CTD_CHECK(ember_event_synchronize(ev[4]));
    if (times) {
      CTD_CHECK(ember_event_elapsed_ms(&times->forward_ms, ev[0], ev[1]));
      CTD_CHECK(ember_event_elapsed_ms(&times->backward_ms, ev[1], ev[2]));
      CTD_CHECK(ember_event_elapsed_ms(&times->clip_ms, ev[2], ev[3]));
      CTD_CHECK(ember_event_elapsed_ms(&times->optimizer_ms, ev[3], ev[4]));
      CTD_CHECK(ember_event_elapsed_ms(&times->total_ms, ev[0], ev[4]));
      times->loss = lv;
      times->grad_norm = gn;
      times->mask_sum = tr->mask_sum;
      times->optimizer_stream_ms = static_cast<float>(tr->opt->offload_stats().last_stream_ms);
    }
    for (auto& e : ev) ember_event_destroy(e);
  });
}

int ctd_trainer_synchronize(ctd_trainer_t t) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (tr->opt) tr->opt->wait_idle();
    runtime::synchronize();
    CTD_CHECK(ember_stream_synchronize(runtime::d2h_stream()));
    CTD_CHECK(ember_stream_synchronize(runtime::h2d_stream()));
  });
}

int ctd_memory_stats(ctd_memory* out) {
  return guarded([&] {
    const DeviceMemoryStats s = device_memory_stats();
    out->allocated = s.allocated_bytes;
    out->peak_allocated = s.peak_allocated_bytes;
    out->reserved = s.reserved_bytes;
    out->peak_reserved = s.peak_reserved_bytes;
    out->pinned_host = pinned_host_bytes();
    size_t fr = 0, tot = 0;
    CTD_CHECK(ember_mem_get_info(&fr, &tot));
    out->device_used = tot - fr;
    out->device_total = tot;
    out->peak_device_used = std::max<uint64_t>(s.peak_device_used_bytes, out->device_used);
    out->device_mallocs = static_cast<uint64_t>(s.num_device_mallocs);
    out->cache_flushes = static_cast<uint64_t>(s.num_cache_flushes);
    out->limit = s.limit_bytes;
  });
}

int ctd_reset_peak_memory(void) {
  return guarded([] { reset_peak_device_memory(); });
}

int ctd_set_device_memory_limit(uint64_t bytes) {
  return guarded([&] { set_device_memory_limit(static_cast<size_t>(bytes)); });
}

int ctd_empty_device_cache(void) {
  return guarded([] { empty_device_cache(); });
}

int ctd_alloc_history_start(void) {
  return guarded([] { start_allocation_history(); });
}

int ctd_alloc_history_mark(const char* label) {
  return guarded([&] { mark_allocation_history(label ? label : ""); });
}

int ctd_alloc_history_stop(const char* path) {
  return guarded([&] {
    if (!path) throw std::runtime_error("null path");
    stop_allocation_history(path);
  });
}

int ctd_alloc_replay(const char* path, uint64_t limit, ctd_alloc_replay_stats* out) {
  return guarded([&] {
    if (!path || !out) throw std::runtime_error("null argument");
    const detail::ArenaStats a = detail::replay_history(path, static_cast<size_t>(limit));
    out->peak_allocated = a.peak_live_bytes;
    out->peak_reserved = a.peak_held_bytes;
    out->reserved_end = a.held_bytes;
    out->segments_obtained = static_cast<uint64_t>(a.segments_obtained);
    out->cache_flushes = static_cast<uint64_t>(a.trims);
  });
}

int ctd_gemm_profile_enable(int32_t on) {
  return guarded([&] { runtime::gemm_profile_enable(on != 0); });
}

int ctd_gemm_profile_collect(ctd_gemm_profile* out) {
  return guarded([&] {
    int64_t l[runtime::kProfileVariants];
    double f[runtime::kProfileVariants], ms[runtime::kProfileVariants];
    runtime::gemm_profile_collect(l, f, ms);
    for (int v = 0; v < runtime::kProfileVariants; ++v) out[v] = ctd_gemm_profile{l[v], f[v], ms[v]};
  });
}

int ctd_trainer_save(ctd_trainer_t t, const char* path) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    runtime::synchronize();
    save_safetensors(tr->named.all, path);
    if (tr->opt) train::save_optimizer_state(*tr->opt, tr->named, train::opt_path_for(path));
  });
}

int ctd_trainer_load(ctd_trainer_t t, const char* path) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    const SafetensorsReader file(path);  // each parameter is read straight into place
    for (auto& [name, p] : tr->named.all) {
      if (!file.find(name)) throw std::runtime_error(std::string("load: ") + path + " lacks " + name);
      file.read(name, p);
    }
    if (tr->opt) train::load_optimizer_state(*tr->opt, tr->named, train::opt_path_for(path));
  });
}

int ctd_trainer_set_lr(ctd_trainer_t t, float lr) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->opt) throw std::runtime_error("no optimizer");
    tr->opt->set_lr(lr);
  });
}

int ctd_trainer_accumulate(ctd_trainer_t t, float scale, float* loss) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!tr->ids.defined()) throw std::runtime_error("no batch set");
    Tensor l = tr->model.forward_train_masked(tr->ids, tr->targets, tr->mask);
    ops::mul_scalar(l, scale).backward();
    if (loss) l.copy_to_host(loss);
  });
}

int ctd_train_run(const char* config_path) {
  return guarded([&] {
    if (!config_path) throw std::runtime_error("null config path");
    train::run(train::load_config(config_path));
  });
}

int ctd_train_lr_at_step(int32_t step, int32_t warmup_steps, int32_t total_steps, float lr,
                         float min_lr_ratio, float* out) {
  return guarded([&] {
    if (!out) throw std::runtime_error("null argument");
    train::Config c;
    c.warmup_steps = warmup_steps;
    c.total_steps = total_steps;
    c.lr = lr;
    c.min_lr_ratio = min_lr_ratio;
    *out = train::lr_at_step(step, c);
  });
}

int ctd_train_host_batch(const char* tok_path, const char* mask_path, int32_t seq_len,
                         const int64_t* docs, int64_t B, int64_t* ids, int64_t* targets,
                         float* mask, float* sum_mask, int64_t* num_docs) {
  return guarded([&] {
    if (!tok_path || !mask_path) throw std::runtime_error("null path");
    const train::DataSplit s = train::load_split(tok_path, mask_path, seq_len);
    if (num_docs) *num_docs = s.num_docs;
    if (B <= 0) return;
    if (!docs || !ids || !targets || !mask) throw std::runtime_error("null argument");
    const train::HostBatch h =
        train::make_host_batch(s, std::vector<int64_t>(docs, docs + B), seq_len);
    std::memcpy(ids, h.input_ids.data(), h.input_ids.size() * sizeof(int64_t));
    std::memcpy(targets, h.targets.data(), h.targets.size() * sizeof(int64_t));
    std::memcpy(mask, h.loss_mask.data(), h.loss_mask.size() * sizeof(float));
    if (sum_mask) *sum_mask = h.sum_mask;
  });
}

int ctd_train_event_json(int32_t step, float loss, float lr, float grad_norm,
                         double tokens_per_sec, double wall_s, int32_t val, char* buf,
                         size_t cap) {
  return guarded([&] {
    const std::string e = val ? train::val_event(step, loss, wall_s)
                              : train::train_event(step, loss, lr, grad_norm, tokens_per_sec, wall_s);
    if (!buf || cap < e.size() + 1) throw std::runtime_error("buffer too small");
    std::memcpy(buf, e.c_str(), e.size() + 1);
  });
}

int ctd_kvcache_create(ctd_trainer_t t, int64_t batch, int64_t max_seq, ctd_kvcache_t* out) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (!out) throw std::runtime_error("null output handle");
    if (batch < 1 || max_seq < 1) throw std::runtime_error("kv cache: batch, max_seq >= 1");
    const nn::LlamaConfig& c = tr->model.config;
    *out = new nn::KVCache(nn::KVCache::allocate(c.num_hidden_layers, c.num_key_value_heads,
                                                 c.head_dim, batch, max_seq, kHIP0));
  });
}

int ctd_kvcache_destroy(ctd_kvcache_t c) {
  return guarded([&] { delete static_cast<nn::KVCache*>(c); });
}

int ctd_kvcache_len(ctd_kvcache_t c, int64_t* current_len) {
  return guarded([&] {
    if (!c) throw std::runtime_error("null kv cache handle");
    *current_len = static_cast<nn::KVCache*>(c)->current_len;
  });
}

int ctd_trainer_forward_cached(ctd_trainer_t t, ctd_kvcache_t cache, const int64_t* ids,
                               int64_t B, int64_t T, int32_t position_start, int32_t last_only,
                               float* logits, int64_t numel) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    Tensor x = Tensor::from_host(ids, {B, T}, DType::kInt64, kHIP0);
    auto* kv = static_cast<nn::KVCache*>(cache);
    Tensor y = last_only ? tr->model.forward_last_logits(x, kv, position_start)
                         : tr->model.forward(x, kv, position_start);
    check_numel(y, numel);
    y.copy_to_host(logits);
  });
}

int ctd_sample(const float* logits, int64_t B, int64_t V, float temperature, int32_t top_k,
               float top_p, uint64_t seed, int32_t draws, int32_t on_device, int64_t* out) {
  return guarded([&] {
    if (B < 0 || V < 1 || draws < 0) throw std::runtime_error("sample: bad sizes");
    Tensor x = Tensor::from_host(logits, {B, 1, V}, DType::kFloat32, on_device ? kHIP0 : kCPU);
    SamplerConfig cfg{temperature, top_k, top_p};
    std::mt19937_64 rng(seed);
    for (int32_t d = 0; d < draws; ++d) {
      const std::vector<int64_t> tok = sample(x, cfg, rng);
      std::copy(tok.begin(), tok.end(), out + static_cast<int64_t>(d) * B);
    }
  });
}

int ctd_trainer_generate(ctd_trainer_t t, const int64_t* prompt, int64_t P, int32_t max_new,
                         float temperature, int32_t top_k, float top_p, uint64_t seed,
                         int64_t max_seq, int64_t* tokens, double* prefill_ms,
                         double* decode_ms) {
  return guarded([&] {
    Trainer* tr = as_trainer(t);
    if (P < 1 || max_new < 0 || P + max_new > max_seq)
      throw std::runtime_error("generate: need 1 <= P and P + max_new <= max_seq");
    generate::Request req;
    req.input_ids.assign(prompt, prompt + P);
    req.max_new_tokens = max_new;
    req.max_seq_len = static_cast<int>(max_seq);
    req.sampler = SamplerConfig{temperature, top_k, top_p};
    req.seed = seed;
    runtime::synchronize();
    int n = 0;
    const generate::LoopResult r =
        generate::generate_loop(tr->model, req, [&](int64_t tok) { tokens[n++] = tok; });
    if (prefill_ms) *prefill_ms = r.prefill_ms;
    if (decode_ms) *decode_ms = r.decode_ms;
  });
}

int ctd_set_head_chunk_rows(int64_t rows) {
  return guarded([&] { ops::set_linear_cross_entropy_chunk_rows(rows); });
}

int ctd_set_head_active_rows(int32_t on) {
  return guarded([&] { ops::set_linear_cross_entropy_active_rows(on != 0); });
}

int ctd_set_attn_ds_bytes(int64_t bytes) {
  return guarded([&] { ops::set_attention_backward_ds_bytes(bytes); });
}

int ctd_set_attn_keep_scores(int32_t on) {
  return guarded([&] { ops::set_attention_keep_scores(on != 0); });
}

}  // extern "C"
