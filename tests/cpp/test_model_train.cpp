// C++-API tests on tiny random models, written as the reference's own tests
// are (tests/test_train_forward.cpp:95-208, tests/test_integration_kvcache.cpp:
// 57-123 of the reference), against include/ctd/ directly.  Run on a GPU by
// tests/test_gpu_cpp.py; the CPU oracle (oracle/ember_oracle.h) pins the
// logits.  Exit status = number of failed tests.
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <functional>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "ctd/autograd.h"
#include "ctd/nn/kv_cache.h"
#include "ctd/nn/model.h"
#include "ctd/ops/attention.h"
#include "ctd/ops/elementwise.h"
#include "ctd/ops/loss.h"
#include "ctd/ops/matmul.h"
#include "ctd/ops/repeat_kv.h"
#include "ctd/optim.h"
#include "ctd/runtime.h"
#include "ctd/safetensors.h"
#include "ctd/tensor.h"
#include "ember_oracle.h"

using namespace ctd;

namespace {

int g_failed = 0;
std::string g_current;

void check(bool ok, const std::string& what) {
  if (!ok) {
    ++g_failed;
    std::printf("  FAILED: %s (in %s)\n", what.c_str(), g_current.c_str());
  }
}

struct TinyCfg {
  int V = 8;
  int D = 8;   // hidden
  int H = 2;   // query heads
  int Hk = 1;  // kv heads
  int Dh = 4;  // head_dim
  int I = 16;
  int L = 1;
  float eps = 1e-5f;
  float theta = 100.0f;
};

Tensor rand_tensor(const std::vector<int64_t>& shape, std::mt19937& rng, float scale,
                   bool grad) {
  std::normal_distribution<float> nd(0.0f, 1.0f);
  int64_t n = 1;
  for (auto d : shape) n *= d;
  std::vector<float> h(static_cast<size_t>(n));
  for (auto& v : h) v = nd(rng) * scale;
  Tensor t = Tensor::from_host(h.data(), shape, DType::kFloat32, kHIP0);
  if (grad) t.requires_grad_(true);
  return t;
}

Tensor linear_w(int64_t out, int64_t in, std::mt19937& rng, bool grad) {
  return rand_tensor({out, in}, rng, 1.0f / std::sqrt(static_cast<float>(in)), grad);
}

Tensor ones_vec(int64_t n, bool grad) {
  std::vector<float> h(static_cast<size_t>(n), 1.0f);
  Tensor t = Tensor::from_host(h.data(), {n}, DType::kFloat32, kHIP0);
  if (grad) t.requires_grad_(true);
  return t;
}

nn::Model build_tiny(const TinyCfg& c, std::mt19937& rng, bool grad) {
  nn::Model m;
  m.config = nn::LlamaConfig{
      .vocab_size = c.V,
      .hidden_size = c.D,
      .intermediate_size = c.I,
      .num_hidden_layers = c.L,
      .num_attention_heads = c.H,
      .num_key_value_heads = c.Hk,
      .head_dim = c.Dh,
      .max_position_embeddings = 64,
      .rms_norm_eps = c.eps,
      .rope_theta = c.theta,
      .tie_word_embeddings = true,
  };
  m.embed_tokens = nn::Embedding{rand_tensor({c.V, c.D}, rng, 0.02f, grad)};
  m.norm = nn::RMSNorm{ones_vec(c.D, grad), c.eps};
  for (int i = 0; i < c.L; ++i) {
    nn::TransformerBlock blk{
        .input_layernorm = {ones_vec(c.D, grad), c.eps},
        .post_attention_layernorm = {ones_vec(c.D, grad), c.eps},
        .self_attn =
            {
                .q_proj = {linear_w(c.H * c.Dh, c.D, rng, grad)},
                .k_proj = {linear_w(c.Hk * c.Dh, c.D, rng, grad)},
                .v_proj = {linear_w(c.Hk * c.Dh, c.D, rng, grad)},
                .o_proj = {linear_w(c.D, c.H * c.Dh, rng, grad)},
                .num_heads = c.H,
                .num_kv_heads = c.Hk,
                .head_dim = c.Dh,
                .rope_theta = c.theta,
            },
        .mlp =
            {
                .gate_proj = {linear_w(c.I, c.D, rng, grad)},
                .up_proj = {linear_w(c.I, c.D, rng, grad)},
                .down_proj = {linear_w(c.D, c.I, rng, grad)},
            },
    };
    m.layers.push_back(std::move(blk));
  }
  return m;
}

std::vector<Tensor> params_of(nn::Model& m) {
  std::vector<Tensor> ps;
  for (auto& [name, t] : m.collect_parameters().all) ps.push_back(t);
  return ps;
}

std::vector<float> host(const Tensor& t) {
  std::vector<float> h(static_cast<size_t>(t.numel()));
  t.copy_to_host(h.data());
  return h;
}

double max_abs_diff(const std::vector<float>& a, const std::vector<float>& b) {
  if (a.size() != b.size()) return INFINITY;
  double m = 0.0;
  for (size_t i = 0; i < a.size(); ++i)
    m = std::max(m, std::abs(static_cast<double>(a[i]) - static_cast<double>(b[i])));
  return m;
}

// Oracle logits [B*T*V] of the model (collect_parameters order).
std::vector<double> oracle_logits(nn::Model& m, const std::vector<int64_t>& ids, int64_t B,
                                  int64_t T) {
  const nn::LlamaConfig& c = m.config;
  orc_cfg oc{};
  oc.vocab = c.vocab_size;
  oc.hidden = c.hidden_size;
  oc.inter = c.intermediate_size;
  oc.layers = c.num_hidden_layers;
  oc.heads = c.num_attention_heads;
  oc.kv_heads = c.num_key_value_heads;
  oc.head_dim = c.head_dim;
  oc.eps = c.rms_norm_eps;
  oc.theta = c.rope_theta;
  oc.rope_factor = c.rope_scaling_factor;
  oc.rope_low_freq = c.rope_scaling_low_freq_factor;
  oc.rope_high_freq = c.rope_scaling_high_freq_factor;
  oc.rope_orig_max_pos = c.rope_scaling_original_max_pos;
  oc.qk_norm = c.qk_norm ? 1 : 0;
  std::vector<std::vector<double>> store;
  std::vector<const double*> ptrs;
  for (const Tensor& p : params_of(m)) {
    std::vector<float> h = host(p);
    store.emplace_back(h.begin(), h.end());
  }
  for (auto& s : store) ptrs.push_back(s.data());
  std::vector<double> out(static_cast<size_t>(B * T * c.vocab_size));
  orc_model_logits(&oc, ptrs.data(), ids.data(), out.data(), B, T);
  return out;
}

void run(const char* name, const std::function<void()>& fn) {
  g_current = name;
  std::printf("[ RUN      ] %s\n", name);
  const int before = g_failed;
  try {
    fn();
  } catch (const std::exception& e) {
    ++g_failed;
    std::printf("  FAILED: exception %s\n", e.what());
  }
  std::printf("[ %s ] %s\n", g_failed == before ? "      OK" : "  FAILED", name);
  std::fflush(stdout);
}

// reference test_train_forward.cpp:138-171 (+ the oracle)
void train_logits_match_inference_logits(TinyCfg c) {
  std::mt19937 rng(42);
  nn::Model m = build_tiny(c, rng, /*grad=*/false);
  std::vector<int64_t> hids = {1, 4, 0, 6, 7, 2, 3, 5};
  for (auto& v : hids) v %= c.V;
  Tensor ids = Tensor::from_host(hids.data(), {2, 4}, DType::kInt64, kHIP0);
  Tensor inf, train;
  {
    autograd::NoGradGuard ng;
    inf = m.forward(ids);
    train = m.forward_train_logits(ids);
  }
  check(inf.shape() == train.shape(), "logit shapes");
  const std::vector<float> a = host(inf), b = host(train);
  check(max_abs_diff(a, b) < 1e-4, "inference vs training logits < 1e-4");
  const std::vector<double> ref = oracle_logits(m, hids, 2, 4);
  double worst = 0.0, scale = 0.0;
  for (size_t i = 0; i < ref.size(); ++i) {
    worst = std::max(worst, std::abs(a[i] - ref[i]));
    scale = std::max(scale, std::abs(ref[i]));
  }
  check(worst <= 1e-4 * scale + 1e-6, "logits vs oracle");
}

// reference test_train_forward.cpp:174-208, also with gradient checkpointing
// and with the offloaded optimizer: the three runs give the same loss bits.
void overfits_tiny_batch() {
  const int B = 2, T = 4;
  std::vector<int64_t> hx = {1, 4, 0, 6, 7, 2, 3, 5};
  std::vector<int64_t> hy = {4, 0, 6, 3, 2, 3, 5, 1};
  std::vector<float> finals;
  for (int variant = 0; variant < 3; ++variant) {
    std::mt19937 rng(123);
    TinyCfg c;
    nn::Model m = build_tiny(c, rng, /*grad=*/true);
    m.gradient_checkpointing = variant >= 1;
    Tensor x = Tensor::from_host(hx.data(), {B, T}, DType::kInt64, kHIP0);
    Tensor y = Tensor::from_host(hy.data(), {B, T}, DType::kInt64, kHIP0);
    optim::AdamW opt(params_of(m), /*lr=*/1e-2f, /*wd=*/0.0f, 0.9f, 0.95f, 1e-8f,
                     /*offload=*/variant == 2);
    constexpr int Steps = 300;
    float first = 0.0f, last = 0.0f;
    for (int step = 0; step < Steps; ++step) {
      opt.zero_grad();
      Tensor loss = m.forward_train(x, y);
      loss.backward();
      opt.step();
      if (step == 0) loss.copy_to_host(&first);
      if (step == Steps - 1) loss.copy_to_host(&last);
    }
    std::printf("  variant %d: first %.5f final %.6f\n", variant, first, last);
    check(first > 1.5f && first < 4.0f, "initial loss near log(8)");
    check(last < 0.05f, "final loss < 0.05");
    finals.push_back(last);
  }
  check(finals[0] == finals[1], "checkpointing leaves the loss bits unchanged");
  check(finals[0] == finals[2], "offloaded AdamW leaves the loss bits unchanged");
}

// The offloaded optimizer's prefetch (started from Model::recompute_hook when
// the backward re-runs layer 0) gives the same weights as no prefetch, also
// when the host state is rewritten through m_tensor() between the backward and
// step() -- as a checkpoint load does -- which must drop the staged copy.
void prefetch_then_host_state_change() {
  const int B = 2, T = 4;
  std::vector<int64_t> hx = {1, 4, 0, 6, 7, 2, 3, 5};
  std::vector<int64_t> hy = {4, 0, 6, 3, 2, 3, 5, 1};
  std::vector<std::vector<float>> finals;
  for (int variant = 0; variant < 2; ++variant) {  // 0: no prefetch, 1: prefetch
    std::mt19937 rng(99);
    TinyCfg c;
    nn::Model m = build_tiny(c, rng, /*grad=*/true);
    m.gradient_checkpointing = true;
    Tensor x = Tensor::from_host(hx.data(), {B, T}, DType::kInt64, kHIP0);
    Tensor y = Tensor::from_host(hy.data(), {B, T}, DType::kInt64, kHIP0);
    optim::AdamW opt(params_of(m), /*lr=*/1e-2f, /*wd=*/0.0f, 0.9f, 0.95f, 1e-8f,
                     /*offload=*/true);
    opt.set_offload_chunk(64);  // the embedding (64 floats) is one chunk of many
    opt.set_prefetch_chunks(variant == 0 ? 0 : 32);
    bool armed = false;
    m.recompute_hook = [&opt, &armed](int layer) {
      if (armed && layer == 0) opt.prefetch();
    };
    for (int step = 0; step < 3; ++step) {
      opt.zero_grad();
      Tensor loss = m.forward_train(x, y);
      armed = true;
      loss.backward();
      armed = false;
      if (step == 1) {  // rewrite the embedding's first moment on the host
        Tensor& mt = opt.m_tensor(0, 0);
        float* hm = static_cast<float*>(mt.data_ptr());
        for (int64_t i = 0; i < mt.numel(); ++i) hm[i] = 0.25f;
      }
      opt.step();
      opt.wait_idle();
      const double pf = opt.offload_stats().last_prefetch_bytes;
      if (variant == 1 && step == 1) check(pf == 0.0, "a rewritten state drops the prefetch");
      if (variant == 1 && step == 2) check(pf > 0.0, "the backward prefetched the embedding's state");
      if (variant == 0) check(pf == 0.0, "no prefetch when switched off");
    }
    m.recompute_hook = nullptr;
    finals.push_back(host(params_of(m)[0]));
  }
  check(finals[0] == finals[1], "prefetch leaves the weights bits unchanged");
}

// The offloaded step moves m/v only for parameters that have a gradient (the
// reference skips the others, src/core/optim.cu:183): with some parameters'
// gradients dropped before each step, the offloaded run equals the on-device
// run bit for bit (weights and m/v), the dropped parameters' state stays zero
// on the host, and exactly their chunks are not transferred.
void offload_skips_state_without_grad() {
  const int B = 2, T = 4;
  std::vector<int64_t> hx = {1, 4, 0, 6, 7, 2, 3, 5};
  std::vector<int64_t> hy = {4, 0, 6, 3, 2, 3, 5, 1};
  TinyCfg c;
  c.L = 2;
  std::vector<std::vector<float>> weights[2], ms[2], vs[2];
  double moved = -1.0, skipped = -1.0;
  int64_t frozen_elems = 0, graded_elems = 0;
  for (int variant = 0; variant < 2; ++variant) {  // 0: on the device, 1: offloaded
    std::mt19937 rng(7);
    nn::Model m = build_tiny(c, rng, /*grad=*/true);
    Tensor x = Tensor::from_host(hx.data(), {B, T}, DType::kInt64, kHIP0);
    Tensor y = Tensor::from_host(hy.data(), {B, T}, DType::kInt64, kHIP0);
    std::vector<Tensor> ps = params_of(m);
    optim::AdamW opt(ps, /*lr=*/1e-2f, /*wd=*/0.1f, 0.9f, 0.95f, 1e-8f, variant == 1);
    opt.set_offload_chunk(64);  // parameters start on 64-float boundaries: one owner per chunk
    opt.set_prefetch_chunks(0);
    // Dropped: every parameter of layer 1 and layer 0's q_proj.
    std::vector<std::string> names;
    for (const auto& [name, t] : m.collect_parameters().all) names.push_back(name);
    auto dropped = [&](size_t i) {
      return names[i].find("layers.1.") != std::string::npos ||
             names[i].find("layers.0.self_attn.q_proj") != std::string::npos;
    };
    for (int step = 0; step < 2; ++step) {
      opt.zero_grad();
      Tensor loss = m.forward_train(x, y);
      loss.backward();
      for (size_t i = 0; i < ps.size(); ++i)
        if (dropped(i)) ps[i].zero_grad_();
      opt.step();
      opt.wait_idle();
    }
    frozen_elems = graded_elems = 0;
    for (size_t i = 0; i < ps.size(); ++i) {
      if (!dropped(i)) graded_elems += ps[i].numel();
      weights[variant].push_back(host(ps[i]));
      ms[variant].push_back(host(opt.m_tensor(0, i)));
      vs[variant].push_back(host(opt.v_tensor(0, i)));
      if (dropped(i)) {
        frozen_elems += (ps[i].numel() + 63) / 64 * 64;
        const auto& mm = ms[variant].back();
        const auto& vv = vs[variant].back();
        check(std::all_of(mm.begin(), mm.end(), [](float f) { return f == 0.0f; }) &&
                  std::all_of(vv.begin(), vv.end(), [](float f) { return f == 0.0f; }),
              "state of a parameter without gradient stays zero");
      }
    }
    if (variant == 1) {
      moved = opt.offload_stats().last_h2d_bytes;
      skipped = opt.offload_stats().last_skipped_bytes;
    }
  }
  check(weights[0] == weights[1], "offloaded weights equal on-device bitwise");
  check(ms[0] == ms[1] && vs[0] == vs[1], "offloaded m/v equal on-device bitwise");
  // Each 64-float chunk holds one parameter (and its padding to 256 bytes):
  // only the elements of parameters with a gradient cross the link, m and v.
  check(moved == 8.0 * static_cast<double>(graded_elems),
        "only parameters with a gradient are moved (" + std::to_string(moved) + " B, expected " +
            std::to_string(8 * graded_elems) + ")");
  check(frozen_elems > 0 && skipped >= 8.0 * static_cast<double>(frozen_elems),
        "the dropped parameters' chunks stay on the host (skipped " + std::to_string(skipped) +
            " B)");
}

// reference test_integration_kvcache.cpp:57-123 on a tiny random model
void kv_cache_equivalences(TinyCfg c) {
  std::mt19937 rng(7);
  nn::Model m = build_tiny(c, rng, /*grad=*/false);
  const int64_t T = 12;
  std::vector<int64_t> hids(T);
  for (int64_t i = 0; i < T; ++i) hids[i] = (3 * i + 1) % c.V;
  Tensor ids = Tensor::from_host(hids.data(), {1, T}, DType::kInt64, kHIP0);
  const std::vector<float> full = host(m.forward(ids));
  {
    nn::KVCache cache = nn::KVCache::allocate(c.L, c.Hk, c.Dh, 1, T + 8, kHIP0);
    const std::vector<float> with = host(m.forward(ids, &cache, 0));
    check(max_abs_diff(full, with) < 5e-5, "prefill with cache == without");
    check(cache.current_len == T, "current_len after prefill");
  }
  nn::KVCache cache = nn::KVCache::allocate(c.L, c.Hk, c.Dh, 1, T + 4, kHIP0);
  Tensor prefix = Tensor::from_host(hids.data(), {1, T - 3}, DType::kInt64, kHIP0);
  (void)m.forward(prefix, &cache, 0);
  for (int64_t t = T - 3; t < T; ++t) {
    Tensor one = Tensor::from_host(&hids[t], {1, 1}, DType::kInt64, kHIP0);
    const std::vector<float> step = host(m.forward(one, &cache, static_cast<int>(t)));
    std::vector<float> row(full.begin() + t * c.V, full.begin() + (t + 1) * c.V);
    check(max_abs_diff(step, row) < 5e-4, "decode step == full-sequence row");
    check(cache.current_len == t + 1, "current_len after decode");
  }
}

// Tensor::backward(..., retain_graph = true) keeps the graph, as the
// reference's engine always does (src/core/autograd.cu:158-237): a second
// pass through it adds the same gradients again (x + x is exact, so every
// gradient is exactly twice the first pass's), through checkpointed layers
// too and through a loss scaled before backward (the fused LM head's node
// then scales into fresh buffers); a last pass without retaining consumes the
// graph, after which another backward throws, as the default always does.
// Attention that keeps its scores, under a retained graph (no checkpointing):
// a retained pass computes S again and leaves the scores intact, so the last,
// consuming pass reads them: its gradients are bitwise those of a fresh
// forward + backward from kept scores, added to the retained passes' sum.
void kept_scores_retained_graph() {
  const int B = 2, T = 70;
  std::mt19937 rng(9);
  TinyCfg c{32, 128, 2, 1, 64, 64, 2, 1e-5f, 1e4f};
  nn::Model m = build_tiny(c, rng, /*grad=*/true);
  std::vector<int64_t> hx(B * T), hy(B * T);
  for (int i = 0; i < B * T; ++i) {
    hx[i] = (i * 7 + 3) % c.V;
    hy[i] = (i * 5 + 1) % c.V;
  }
  Tensor x = Tensor::from_host(hx.data(), {B, T}, DType::kInt64, kHIP0);
  Tensor y = Tensor::from_host(hy.data(), {B, T}, DType::kInt64, kHIP0);
  std::vector<Tensor> ps = params_of(m);
  struct Keep {
    Keep() { ops::set_attention_keep_scores(true); }
    ~Keep() { ops::set_attention_keep_scores(false); }
  } keep;
  m.forward_train(x, y).backward();
  std::vector<std::vector<float>> gk;
  for (Tensor& p : ps) {
    gk.push_back(host(p.grad()));
    p.zero_grad_();
  }
  Tensor loss = m.forward_train(x, y);
  loss.backward(/*retain_graph=*/true);
  std::vector<std::vector<float>> g1;
  for (Tensor& p : ps) g1.push_back(host(p.grad()));
  loss.backward(/*retain_graph=*/true);
  loss.backward();
  bool exact = true;
  double num = 0.0, den = 0.0;
  for (size_t i = 0; i < ps.size(); ++i) {
    const std::vector<float> g3 = host(ps[i].grad());
    for (size_t j = 0; j < g3.size(); ++j) {
      const float two = g1[i][j] + g1[i][j];
      exact = exact && g3[j] == two + gk[i][j];
      num += (gk[i][j] - g1[i][j]) * static_cast<double>(gk[i][j] - g1[i][j]);
      den += static_cast<double>(g1[i][j]) * g1[i][j];
    }
  }
  check(exact, "the consuming pass reads the scores the retained passes left intact");
  check(std::sqrt(num / den) < 1e-5, "kept-score gradients agree with the recompute path");
}

void retained_graph_repeat_backward(bool checkpointing, float upstream) {
  const int B = 2, T = 6;
  std::vector<int64_t> hx = {1, 4, 0, 6, 7, 2, 3, 5, 2, 2, 1, 0};
  std::vector<int64_t> hy = {4, 0, 6, 3, 2, 3, 5, 1, 7, 6, 5, 4};
  std::mt19937 rng(7);
  TinyCfg c{32, 128, 2, 1, 64, 64, 2, 1e-5f, 1e4f};
  nn::Model m = build_tiny(c, rng, /*grad=*/true);
  m.gradient_checkpointing = checkpointing;
  Tensor x = Tensor::from_host(hx.data(), {B, T}, DType::kInt64, kHIP0);
  Tensor y = Tensor::from_host(hy.data(), {B, T}, DType::kInt64, kHIP0);
  std::vector<Tensor> ps = params_of(m);

  Tensor loss = m.forward_train(x, y);
  Tensor root = upstream == 1.0f ? loss : ops::mul_scalar(loss, upstream);
  root.backward(/*retain_graph=*/true);
  std::vector<std::vector<float>> g1;
  for (Tensor& p : ps) g1.push_back(host(p.grad()));
  root.backward(/*retain_graph=*/true);
  bool doubled = true;
  for (size_t i = 0; i < ps.size(); ++i) {
    const std::vector<float> g2 = host(ps[i].grad());
    for (size_t j = 0; j < g2.size(); ++j) doubled = doubled && g2[j] == 2.0f * g1[i][j];
  }
  check(doubled, "second pass through the retained graph doubles every gradient");
  root.backward();  // consumes the graph
  double worst = 0.0;
  for (size_t i = 0; i < ps.size(); ++i) {
    const std::vector<float> g3 = host(ps[i].grad());
    for (size_t j = 0; j < g3.size(); ++j)
      worst = std::max(worst, std::abs(static_cast<double>(g3[j]) - 3.0 * g1[i][j]) /
                                  (1e-30 + std::abs(3.0 * g1[i][j])));
  }
  check(worst < 1e-6, "third pass adds the same gradients once more");
  bool threw = false;
  try {
    root.backward();
  } catch (const std::runtime_error&) {
    threw = true;
  }
  check(threw, "a consumed graph refuses another backward");

  // The default (no retain) consumes the graph on its first pass.
  for (Tensor& p : ps) p.zero_grad_();
  Tensor l2 = m.forward_train(x, y);
  l2.backward();
  threw = false;
  try {
    l2.backward();
  } catch (const std::runtime_error&) {
    threw = true;
  }
  check(threw, "default backward consumes the graph");
  if (upstream == 1.0f) {  // and gives the first retained pass's gradients
    bool same = true;
    for (size_t i = 0; i < ps.size(); ++i) same = same && host(ps[i].grad()) == g1[i];
    check(same, "retained and default passes give the same gradients");
  }
}

// optim::SGD (the reference's include/ctd/optim.h:11-20): p <- p - lr * g for
// parameters with a gradient, untouched otherwise; zero_grad drops the grads;
// a parameter that does not require grad is rejected.
void sgd_step() {
  std::mt19937 rng(3);
  Tensor a = rand_tensor({300}, rng, 1.0f, true);
  Tensor b = rand_tensor({17}, rng, 1.0f, true);
  const std::vector<float> a0 = host(a), b0 = host(b);
  // y = a * c with a constant c: backward(ones) leaves a.grad = c
  std::vector<float> ga(300);
  for (size_t i = 0; i < 300; ++i) ga[i] = 0.5f * static_cast<float>(i % 7) - 1.0f;
  const std::vector<float> ones(300, 1.0f);
  ops::mul(a, Tensor::from_host(ga.data(), {300}, DType::kFloat32, kHIP0))
      .backward(Tensor::from_host(ones.data(), {300}, DType::kFloat32, kHIP0));
  optim::SGD opt({a, b}, 0.1f);
  opt.step();
  const std::vector<float> a1 = host(a), b1 = host(b);
  bool ok = true;
  for (size_t i = 0; i < 300; ++i) ok = ok && a1[i] == std::fma(-0.1f, ga[i], a0[i]);
  check(ok, "SGD: fma(-lr, g, p), one rounding");
  check(b1 == b0, "SGD: parameters without a gradient are untouched");
  opt.zero_grad();
  check(!a.grad().storage(), "SGD: zero_grad drops the gradient");
  Tensor c = rand_tensor({4}, rng, 1.0f, false);
  bool threw = false;
  try {
    optim::SGD bad({c}, 0.1f);
  } catch (const std::runtime_error&) {
    threw = true;
  }
  check(threw, "SGD: a parameter without requires_grad is rejected");
}

// ------------------------------------------------------------ safetensors
namespace fs = std::filesystem;

void write_raw(const fs::path& p, const std::string& header, size_t data_bytes) {
  std::ofstream f(p, std::ios::binary);
  const uint64_t n = header.size();
  f.write(reinterpret_cast<const char*>(&n), 8);
  f.write(header.data(), static_cast<std::streamsize>(n));
  const std::string data(data_bytes, '\0');
  f.write(data.data(), static_cast<std::streamsize>(data.size()));
}

bool throws_with(const std::function<void()>& fn, const std::string& needle) {
  try {
    fn();
  } catch (const std::runtime_error& e) {
    if (std::string(e.what()).find(needle) != std::string::npos) return true;
    std::printf("    message was: %s\n", e.what());
    return false;
  }
  return false;
}

// The writer's header for two tensors inserted as b then a, written out by
// hand: keys sorted, fields data_offsets / dtype / shape, no spaces, offsets in
// insertion order, padded with spaces to a multiple of 8 (110 -> 112 bytes).
void safetensors_format_and_faults(Device dev) {
  const fs::path dir = fs::temp_directory_path() /
                       ("ctd_st_" + std::to_string(::getpid()) + (dev.is_hip() ? "_d" : "_h"));
  fs::create_directories(dir);
  const float b_vals[2] = {1.0f, 2.0f}, a_vals[2] = {3.0f, -4.5f};
  const std::vector<std::pair<std::string, Tensor>> items = {
      {"b", Tensor::from_host(b_vals, {2}, DType::kFloat32, dev)},
      {"a", Tensor::from_host(a_vals, {1, 2}, DType::kFloat32, dev)}};
  const fs::path file = dir / "two.safetensors";
  save_safetensors(items, file);
  const std::string want =
      "{\"a\":{\"data_offsets\":[8,16],\"dtype\":\"F32\",\"shape\":[1,2]},"
      "\"b\":{\"data_offsets\":[0,8],\"dtype\":\"F32\",\"shape\":[2]}}  ";
  {
    std::ifstream f(file, std::ios::binary);
    uint64_t n = 0;
    f.read(reinterpret_cast<char*>(&n), 8);
    std::string head(n, '\0');
    f.read(head.data(), static_cast<std::streamsize>(n));
    float data[4];
    f.read(reinterpret_cast<char*>(data), sizeof data);
    check(n == 112 && head == want, "header bytes");
    check(data[0] == 1.0f && data[1] == 2.0f && data[2] == 3.0f && data[3] == -4.5f,
          "data in insertion order");
    check(fs::file_size(file) == 8 + 112 + 16, "file size");
  }
  TensorDict back = load_safetensors(file, dev);
  std::vector<float> got(2);
  back.at("a").copy_to_host(got.data());
  check(back.size() == 2 && back.at("a").shape() == std::vector<int64_t>{1, 2} &&
            got[0] == 3.0f && got[1] == -4.5f,
        "round trip");
  {  // SafetensorsReader::read into caller memory
    SafetensorsReader r(file);
    Tensor dst = Tensor::zeros({2}, DType::kFloat32, dev);
    r.read("b", dst);
    dst.copy_to_host(got.data());
    check(got[0] == 1.0f && got[1] == 2.0f && r.find("c") == nullptr, "reader read");
    Tensor wrong = Tensor::zeros({3}, DType::kFloat32, dev);
    check(throws_with([&] { r.read("b", wrong); }, "destination differs"), "reader shape check");
  }
  const std::string ok_entry = "\"x\":{\"dtype\":\"F32\",\"shape\":[2],\"data_offsets\":[0,8]}";
  struct Bad {
    const char* what;
    std::string header;
    size_t data;
    const char* needle;
  };
  const Bad bad[] = {
      {"bad JSON", "{\"x\":", 8, "malformed header"},
      {"range past the data", "{" + ok_entry + "}", 4, "inconsistent layout"},
      {"size vs shape", "{\"x\":{\"dtype\":\"F32\",\"shape\":[3],\"data_offsets\":[0,8]}}", 8,
       "inconsistent layout"},
      {"overlap", "{" + ok_entry + ",\"y\":{\"dtype\":\"F32\",\"shape\":[1],\"data_offsets\":[4,8]}}",
       8, "overlap"},
      {"F16", "{\"x\":{\"dtype\":\"F16\",\"shape\":[4],\"data_offsets\":[0,8]}}", 8,
       "unsupported dtype"},
      {"negative extent", "{\"x\":{\"dtype\":\"F32\",\"shape\":[-2],\"data_offsets\":[0,8]}}", 8,
       "malformed header"},
      // Products that wrap 64 bits to 0 must not pass as an empty tensor.
      {"element count wraps",
       "{\"x\":{\"dtype\":\"F32\",\"shape\":[8589934592,2147483648],\"data_offsets\":[0,0]}}", 8,
       "too large to address"},
      {"byte count wraps",
       "{\"x\":{\"dtype\":\"F32\",\"shape\":[4611686018427387904],\"data_offsets\":[0,0]}}", 8,
       "too large to address"},
      {"extent past int64",
       "{\"x\":{\"dtype\":\"F32\",\"shape\":[9223372036854775808,0],\"data_offsets\":[0,0]}}", 8,
       "too large to address"},
  };
  for (const Bad& b : bad) {
    const fs::path p = dir / "bad.safetensors";
    write_raw(p, b.header, b.data);
    check(throws_with([&] { load_safetensors(p, dev); }, b.needle), b.what);
  }
  {  // header length larger than the file
    const fs::path p = dir / "short.safetensors";
    std::ofstream f(p, std::ios::binary);
    const uint64_t n = 1000;
    f.write(reinterpret_cast<const char*>(&n), 8);
    f << "{}";
    f.close();
    check(throws_with([&] { load_safetensors(p, dev); }, "truncated file"), "truncated");
  }
  check(throws_with([&] { load_safetensors(dir / "missing.safetensors", dev); }, "cannot open"),
        "missing file");
  const int64_t ids[2] = {1, 2};
  check(throws_with([&] {
          save_safetensors({{"i", Tensor::from_host(ids, {2}, DType::kInt64, dev)}}, dir / "i.st");
        }, "F32 tensors only"),
        "writer dtype");
  check(!fs::exists(dir / "i.st") && !fs::exists(dir / "i.st.partial"), "no partial file left");
  fs::remove_all(dir);
}

// The recompute form of a block (TransformerBlock::forward_train_for_backward)
// records the graph of the block's output without computing its last GEMM
// and residual add: back-propagating an upstream gradient through it must
// give every gradient of forward_train bit for bit, and its result must be
// h's storage, values untouched.
void block_graph_only_recompute_matches_forward_train() {
  TinyCfg c{32, 128, 2, 1, 64, 64, 1, 1e-5f, 1e4f};
  std::mt19937 rng(11);
  nn::Model m = build_tiny(c, rng, true);
  const nn::TransformerBlock& blk = m.layers[0];
  const int64_t B = 2, T = 24;
  Tensor x0 = rand_tensor({B, T, c.D}, rng, 1.0f, false);
  Tensor dy = rand_tensor({B, T, c.D}, rng, 1.0f, false);
  auto params = [&] {
    const auto& a = blk.self_attn;
    return std::vector<Tensor>{blk.input_layernorm.weight, blk.post_attention_layernorm.weight,
                               a.q_proj.weight, a.k_proj.weight, a.v_proj.weight,
                               a.o_proj.weight, blk.mlp.gate_proj.weight,
                               blk.mlp.up_proj.weight, blk.mlp.down_proj.weight};
  };
  auto run_once = [&](bool graph_only, std::vector<float>* y_host) {
    for (auto& p : params()) p.zero_grad_();
    Tensor x = x0.detach();
    x.requires_grad_(true);
    Tensor y = graph_only ? blk.forward_train_for_backward(x) : blk.forward_train(x);
    if (y_host && !graph_only) *y_host = host(y);
    if (graph_only) {
      // Its elements are not the block output: reading them throws, the
      // graph is still there for backward.
      check(y.is_placeholder(), "the recompute form is a placeholder");
      check(throws_with([&] { (void)y.data_ptr(); }, "autograd history"),
            "data_ptr() of the recompute form throws");
      check(throws_with([&] { std::vector<float> t(y.numel()); y.copy_to_host(t.data()); },
                        "autograd history"),
            "copy_to_host() of the recompute form throws");
      check(throws_with([&] { (void)y.reshape({-1}).data_ptr(); }, "autograd history"),
            "a view of the recompute form throws too");
      check(y.autograd_meta() && y.autograd_meta()->grad_fn, "the recompute form keeps its grad_fn");
    }
    y.backward(dy);
    std::vector<std::vector<float>> g{host(x.grad())};
    for (auto& p : params()) g.push_back(host(p.grad()));
    return g;
  };
  std::vector<float> y_full;
  const auto g_full = run_once(false, &y_full);
  const auto g_graph = run_once(true, nullptr);
  check(g_full.size() == g_graph.size(), "same gradient count");
  for (size_t i = 0; i < g_full.size() && i < g_graph.size(); ++i)
    check(g_full[i] == g_graph[i], "gradient " + std::to_string(i) + " bitwise equal");
  check(!y_full.empty(), "forward_train's output is readable");

  // ops-level: the result is a view of `values`, which are left as they were.
  Tensor a2 = rand_tensor({5, 8}, rng, 1.0f, true), w = rand_tensor({3, 8}, rng, 1.0f, true);
  Tensor vals = rand_tensor({15}, rng, 1.0f, false);
  const std::vector<float> before = host(vals);
  Tensor y2 = ops::matmul_graph_only(a2, w, false, true, vals);
  check(y2.shape() == std::vector<int64_t>{5, 3}, "matmul_graph_only shape");
  check(y2.storage() == vals.storage() && host(vals) == before, "matmul_graph_only is a view");
  check(y2.is_placeholder() && throws_with([&] { (void)y2.data_ptr(); }, "autograd history"),
        "matmul_graph_only's result cannot be read");
  check(!vals.is_placeholder(), "the values tensor itself stays readable");
  check(throws_with([&] { ops::matmul_graph_only(a2, w, false, true, a2); }, "M*N"),
        "matmul_graph_only rejects values of another size");
}

// A matmul whose input already holds another consumer's gradient adds its
// own into it inside the GEMM (beta = 1).  The input gradient must be bitwise
// what the engine's separate adds give when each product reads its own view
// of x (so nothing can be folded), for an unsplit and a split-K product.
void fan_in_fold_matches_separate_adds() {
  std::mt19937 rng(12);
  for (int64_t O : {96, 2048}) {
    const int64_t N = 300, K = 64;
    Tensor x0 = rand_tensor({N, K}, rng, 1.0f, false);
    Tensor w1 = rand_tensor({O, K}, rng, 0.1f, false), w2 = rand_tensor({O, K}, rng, 0.1f, false),
           w3 = rand_tensor({O, K}, rng, 0.1f, false);
    Tensor dy = rand_tensor({N, O}, rng, 1.0f, false);
    auto run_once = [&](bool shared) {
      Tensor x = x0.detach();
      x.requires_grad_(true);
      auto view = [&] { return shared ? x : x.reshape({N, K}); };
      Tensor y = ops::add(ops::add(ops::matmul(view(), w1, false, true),
                                   ops::matmul(view(), w2, false, true)),
                          ops::matmul(view(), w3, false, true));
      y.backward(dy);
      return host(x.grad());
    };
    const std::vector<float> folded = run_once(true), separate = run_once(false);
    check(folded == separate, "fan-in folded into the GEMM is bitwise the separate adds, O = " +
                                  std::to_string(O));
  }
  // The residual stream: an RMSNorm's dx added into x's running sum.
  for (int64_t H : {128, 2048, 130}) {
    const int64_t N = 77;
    Tensor x0 = rand_tensor({N, H}, rng, 1.0f, false);
    Tensor w = rand_tensor({H}, rng, 0.1f, false);
    Tensor dy = rand_tensor({N, H}, rng, 1.0f, false);
    auto run_once = [&](bool shared) {
      Tensor x = x0.detach();
      x.requires_grad_(true);
      Tensor xn = shared ? x : x.reshape({N, H});
      Tensor y = ops::add(ops::rms_norm(xn, w, 1e-6f), x);
      y.backward(dy);
      return host(x.grad());
    };
    const std::vector<float> folded = run_once(true), separate = run_once(false);
    check(folded == separate, "RMSNorm dx folded into the running sum is bitwise the separate "
                              "add, H = " + std::to_string(H));
  }
}

}  // namespace


// The reference's masked CE offsets the logits by an int32 row * V
// (src/ops/loss.cu:263-264, 322-323), which wraps once row * V passes 2^31:
// row 14134 straddles it at V = 151936 (its first element sits at
// 2,147,463,424, its last past 2^31) and every later row starts beyond it.
// Through ops::cross_entropy_masked and its backward, N = 14200 rows
// (2.16e9 logits, 8.6 GB): the loss over all rows, and dlogits of rows on
// both sides of the wrap, against the oracle.  Row r holds pattern row r % 16,
// so the oracle needs only the 16 pattern rows for the loss.
void ce_masked_past_int32() {
  const int64_t N = 14200, V = 151936, P = 16;
  std::mt19937 rng(5);
  std::normal_distribution<float> nd(0.0f, 2.0f);
  std::vector<float> pat(static_cast<size_t>(P * V));
  for (auto& x : pat) x = nd(rng);
  std::vector<int64_t> tg(N);
  std::vector<float> mask(N);
  for (int64_t r = 0; r < N; ++r) {
    tg[r] = (r * 7919 + 13) % V;
    mask[r] = r % 7 == 3 ? 0.0f : 1.0f;
  }
  Tensor logits = Tensor::empty({N, V}, DType::kFloat32, kHIP0);
  {
    Tensor rows = Tensor::from_host(pat.data(), {P, V}, DType::kFloat32, kHIP0);
    auto copy_rows = [&](const void* src, int64_t row0, int64_t n) {
      CTD_CHECK(ember_memcpy_async(static_cast<float*>(logits.data_ptr()) + row0 * V, src,
                                   static_cast<size_t>(n * V) * sizeof(float), 2,
                                   runtime::compute_stream()));
    };
    copy_rows(rows.data_ptr(), 0, P);
    for (int64_t filled = P; filled < N;) {  // doubling copies of the rows so far
      const int64_t n = std::min(filled, N - filled);
      copy_rows(logits.data_ptr(), filled, n);
      filled += n;
    }
    runtime::synchronize();
  }
  logits.requires_grad_(true);
  Tensor t = Tensor::from_host(tg.data(), {N}, DType::kInt64, kHIP0);
  Tensor m = Tensor::from_host(mask.data(), {N}, DType::kFloat32, kHIP0);
  Tensor loss = ops::cross_entropy_masked(logits, t, m);
  float got = 0.0f;
  loss.copy_to_host(&got);

  // Oracle: lse of each pattern row, then sum over rows of mask*(lse - logit[t]).
  std::vector<double> patd(pat.begin(), pat.end()), lse(P);
  std::vector<int64_t> zero_t(P, 0);
  std::vector<double> ones(P, 1.0);
  orc_ce_masked_fwd(patd.data(), zero_t.data(), ones.data(), P, V, lse.data(), nullptr);
  double num = 0.0, den = 0.0;
  for (int64_t r = 0; r < N; ++r) {
    if (mask[r] == 0.0f) continue;
    num += lse[r % P] - patd[static_cast<size_t>((r % P) * V + tg[r])];
    den += 1.0;
  }
  const double ref = num / den;
  check(std::abs(got - ref) <= 1e-4 * std::abs(ref), "loss over 2.16e9 logits vs oracle (" +
                                                          std::to_string(got) + " vs " +
                                                          std::to_string(ref) + ")");

  loss.backward();
  Tensor g = logits.grad();
  check(g.defined() && g.shape() == logits.shape(), "dlogits shape");
  for (int64_t r : {int64_t{0}, int64_t{3}, int64_t{14133}, int64_t{14134}, int64_t{14135},
                    int64_t{14136}, int64_t{N - 1}}) {
    std::vector<float> row(V);
    g.view_at(r * V, {V}).copy_to_host(row.data());
    std::vector<double> ref_row(V);
    const double one = 1.0;
    const int64_t tr = tg[r];
    orc_ce_masked_bwd(patd.data() + (r % P) * V, &tr, &one, 1, V, mask[r] / den, ref_row.data());
    double worst = 0.0, scale = 0.0;
    for (int64_t j = 0; j < V; ++j) {
      worst = std::max(worst, std::abs(row[j] - ref_row[j]));
      scale = std::max(scale, std::abs(ref_row[j]));
    }
    if (mask[r] == 0.0f)
      check(worst == 0.0, "masked row " + std::to_string(r) + " has zero dlogits");
    else
      check(worst <= 1e-4 * scale, "dlogits row " + std::to_string(r) + " vs oracle (max err " +
                                       std::to_string(worst) + ", scale " +
                                       std::to_string(scale) + ")");
  }
}

// The MLP's memory-saving forms give the bits of the plain ones: the SwiGLU
// backward writing its gradients over gate and up (when the node holds them
// alone), the down projection's dW before its dA (its input's memory then
// holds dA), and the no-grad activation written over the gate's buffer.
void mlp_in_place_forms_match() {
  std::mt19937 rng(21);
  const int64_t N = 300, H = 96, I = 256;
  Tensor x0 = rand_tensor({N, H}, rng, 1.0f, false);
  Tensor wg = rand_tensor({I, H}, rng, 0.1f, true), wu = rand_tensor({I, H}, rng, 0.1f, true),
         wd = rand_tensor({H, I}, rng, 0.1f, true);
  Tensor dy = rand_tensor({N, H}, rng, 1.0f, false);
  auto run_once = [&](bool hold) {
    wg.zero_grad_();
    wu.zero_grad_();
    wd.zero_grad_();
    Tensor x = x0.detach();
    x.requires_grad_(true);
    Tensor g = ops::matmul(x, wg, false, true), u = ops::matmul(x, wu, false, true);
    std::vector<float> g_before = host(g), u_before = host(u);
    Tensor y = ops::matmul(ops::swiglu(g, u), wd, false, true);
    Tensor keep_g = hold ? g : Tensor{}, keep_u = hold ? u : Tensor{};
    g = Tensor{};
    u = Tensor{};
    y.backward(dy);
    if (hold)
      check(host(keep_g) == g_before && host(keep_u) == u_before,
            "gate and up held by the caller are not overwritten by the backward");
    return std::vector<std::vector<float>>{host(x.grad()), host(wg.grad()), host(wu.grad()),
                                           host(wd.grad())};
  };
  const auto in_place = run_once(false), held = run_once(true);
  check(in_place == held, "gradients with gate/up overwritten equal the out-of-place ones");

  nn::MLP mlp{nn::Linear{wg.detach()}, nn::Linear{wu.detach()}, nn::Linear{wd.detach()}};
  std::vector<float> fused, plain;
  {
    autograd::NoGradGuard ng;
    fused = host(mlp.activation(x0));
    plain = host(ops::swiglu(ops::matmul(x0, wg, false, true), ops::matmul(x0, wu, false, true)));
  }
  check(fused == plain, "no-grad activation over the gate's buffer equals swiglu()");
  bool threw = false;
  try {
    Tensor g = ops::matmul(x0, wg, false, true);  // requires grad through wg
    ops::swiglu_(g, ops::matmul(x0, wu, false, true));
  } catch (const std::runtime_error&) {
    threw = true;
  }
  check(threw, "swiglu_ refuses tensors that require grad");
}

int main(int argc, char** argv) {
  // --cpu: only the tests that need no GPU (host tensors only).
  if (argc > 1 && std::strcmp(argv[1], "--cpu") == 0) {
    run("Safetensors.FormatAndFaults_Host", [] { safetensors_format_and_faults(kCPU); });
    std::printf("%d failure(s)\n", g_failed);
    return g_failed;
  }
  // --large: the test that needs ~18 GB of device memory, on its own.
  if (argc > 1 && std::strcmp(argv[1], "--large") == 0) {
    run("Loss.CrossEntropyMaskedPastInt32Offsets", [] { ce_masked_past_int32(); });
    std::printf("%d failure(s)\n", g_failed);
    return g_failed;
  }
  run("Safetensors.FormatAndFaults_Host", [] { safetensors_format_and_faults(kCPU); });
  run("Safetensors.FormatAndFaults_Device", [] { safetensors_format_and_faults(kHIP0); });
  run("Optim.SGD", [] { sgd_step(); });
  run("Autograd.BlockGraphOnlyRecompute",
      [] { block_graph_only_recompute_matches_forward_train(); });
  run("Autograd.FanInFoldMatchesSeparateAdds", [] { fan_in_fold_matches_separate_adds(); });
  run("Ops.MLPInPlaceFormsMatch", [] { mlp_in_place_forms_match(); });
  run("Autograd.RetainedGraphRepeatBackward", [] { retained_graph_repeat_backward(false, 1.0f); });
  run("Autograd.RetainedGraphRepeatBackward_Checkpointed",
      [] { retained_graph_repeat_backward(true, 1.0f); });
  run("Autograd.RetainedGraphRepeatBackward_ScaledLoss",
      [] { retained_graph_repeat_backward(true, 0.25f); });
  // The same with attention keeping its scores: a retained pass computes S
  // again and leaves the scores for the last, consuming pass.
  run("Autograd.RetainedGraphKeptScores", [] { kept_scores_retained_graph(); });
  run("Autograd.RetainedGraphRepeatBackward_Checkpointed_KeptScores", [] {
    // each pass re-runs the blocks, whose attention keeps fresh scores that
    // the re-run's own (consuming) backward reads: the same path every pass
    struct Keep {
      Keep() { ops::set_attention_keep_scores(true); }
      ~Keep() { ops::set_attention_keep_scores(false); }
    } keep;
    retained_graph_repeat_backward(true, 1.0f);
  });
  run("ModelTrain.TrainLogitsMatchInferenceLogits",
      [] { train_logits_match_inference_logits(TinyCfg{}); });
  run("ModelTrain.TrainLogitsMatchInferenceLogits_D64",
      [] { train_logits_match_inference_logits(TinyCfg{32, 128, 2, 1, 64, 64, 2, 1e-5f, 1e4f}); });
  run("ModelTrain.OverfitsTinyBatch", [] { overfits_tiny_batch(); });
  run("Optim.PrefetchThenHostStateChange", [] { prefetch_then_host_state_change(); });
  run("Optim.OffloadSkipsStateWithoutGrad", [] { offload_skips_state_without_grad(); });
  run("Integration.KVCacheEquivalences", [] { kv_cache_equivalences(TinyCfg{}); });
  run("Integration.KVCacheEquivalences_D64",
      [] { kv_cache_equivalences(TinyCfg{32, 128, 2, 1, 64, 64, 2, 1e-5f, 1e4f}); });
  std::printf("%d failure(s)\n", g_failed);
  return g_failed;
}
