// Token generation behind the ctd_generate protocol.
// Reference: tools/ctd_generate/main.cpp:52-192 (request fields and defaults,
// stop reasons, budget forcing, reply lines).
//
// Differences that keep the protocol: the prefill runs the LM head on the last
// position only (Model::forward_last_logits; the reference computes [1, T, V]
// logits and copies all of them to the host to keep the last row), and greedy
// steps take the argmax on the device.
#include "ctd/generate.h"

#include <algorithm>
#include <chrono>
#include <random>
#include <stdexcept>
#include <unordered_set>

#include "ctd/nn/kv_cache.h"
#include "ctd/nn/model.h"
#include "ctd/runtime.h"
#include "ctd/safetensors.h"
#include "ctd/train.h"
#include "ember_hip.h"
#include "json.h"

namespace ctd::generate {

namespace {

using json::JVal;

double number(const JVal& v, const std::string& key) {
  if (v.kind != JVal::kNum) throw std::runtime_error("request: " + key + " must be a number");
  return v.num;
}

int64_t integer(const JVal& v, const std::string& key) {
  if (v.kind != JVal::kNum) throw std::runtime_error("request: " + key + " must be an integer");
  if (v.str.find_first_of(".eE") == std::string::npos) return std::stoll(v.str);
  return static_cast<int64_t>(v.num);
}

std::vector<int64_t> ids(const JVal& v, const std::string& key) {
  std::vector<int64_t> out;
  if (v.kind == JVal::kNum) {  // a lone id counts as a one-element list
    out.push_back(integer(v, key));
    return out;
  }
  if (v.kind != JVal::kArr) throw std::runtime_error("request: " + key + " must be a list");
  for (const JVal& e : v.arr) out.push_back(integer(e, key));
  return out;
}

std::string line(const json::ObjectWriter& w) { return w.str() + "\n"; }

double seconds_since(std::chrono::steady_clock::time_point t) {
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t).count();
}

}  // namespace

Request parse_request(const std::string& text) {
  const JVal req = json::Parser(text, "request: bad JSON").parse();
  if (req.kind != JVal::kObj) throw std::runtime_error("request: expected a JSON object");
  Request r;
  r.input_ids = ids(req.at("input_ids"), "input_ids");
  if (const JVal* v = req.find("max_new_tokens"))
    r.max_new_tokens = static_cast<int>(integer(*v, "max_new_tokens"));
  if (const JVal* v = req.find("max_seq_len"))
    r.max_seq_len = static_cast<int>(integer(*v, "max_seq_len"));
  if (const JVal* v = req.find("temperature"))
    r.sampler.temperature = static_cast<float>(number(*v, "temperature"));
  if (const JVal* v = req.find("top_k")) r.sampler.top_k = static_cast<int>(integer(*v, "top_k"));
  if (const JVal* v = req.find("top_p"))
    r.sampler.top_p = static_cast<float>(number(*v, "top_p"));
  if (const JVal* v = req.find("seed")) {
    if (v->kind != JVal::kNum) throw std::runtime_error("request: seed must be an integer");
    r.seed = v->str.find_first_of(".eE-") == std::string::npos
                 ? std::stoull(v->str)
                 : static_cast<uint64_t>(integer(*v, "seed"));
  }
  if (const JVal* v = req.find("eos_ids")) r.eos_ids = ids(*v, "eos_ids");
  if (const JVal* v = req.find("thinking_token_budget"))
    r.thinking_token_budget = static_cast<int>(integer(*v, "thinking_token_budget"));
  if (const JVal* v = req.find("think_open_ids")) r.think_open_ids = ids(*v, "think_open_ids");
  if (const JVal* v = req.find("think_close_ids")) r.think_close_ids = ids(*v, "think_close_ids");
  return r;
}

ThinkBudget::ThinkBudget(const Request& r)
    : active_(r.thinking_token_budget > 0 && !r.think_open_ids.empty() &&
              !r.think_close_ids.empty()),
      budget_(r.thinking_token_budget),
      open_(r.think_open_ids),
      close_(r.think_close_ids),
      cap_(std::max(r.think_open_ids.size(), r.think_close_ids.size())) {}

bool ThinkBudget::next_forced(int64_t* tok) {
  if (!active_ || queue_.empty()) return false;
  *tok = queue_.front();
  queue_.erase(queue_.begin());
  return true;
}

bool ThinkBudget::ends_with(const std::vector<int64_t>& seq) const {
  return window_.size() >= seq.size() &&
         std::equal(seq.begin(), seq.end(), window_.end() - static_cast<int64_t>(seq.size()));
}

void ThinkBudget::observe(int64_t tok) {
  if (!active_) return;
  window_.push_back(tok);
  if (window_.size() > cap_) window_.erase(window_.begin());
  if (ends_with(open_)) {
    in_think_ = true;
    count_ = 0;
  } else if (ends_with(close_)) {
    in_think_ = false;
  } else if (in_think_) {
    ++count_;
  }
  if (in_think_ && queue_.empty() && count_ >= budget_) queue_ = close_;
}

namespace {

// Greedy token choice on the device into `out` (int64 [1]), no host sync.
void device_argmax(const Tensor& last, Tensor& out) {
  const int64_t V = last.shape().back();
  const size_t wsb = ember_argmax_rows_workspace_bytes(1, V);
  Tensor ws = wsb ? Tensor::empty({static_cast<int64_t>((wsb + 7) / 8)}, DType::kInt64, kHIP0)
                  : Tensor{};
  CTD_CHECK(ember_argmax_rows_ws(static_cast<const float*>(last.data_ptr()), 1, V,
                                 static_cast<int64_t*>(out.data_ptr()),
                                 wsb ? ws.data_ptr() : nullptr, wsb, runtime::compute_stream()));
}

class Event {
 public:
  Event() { CTD_CHECK(ember_event_create(&e_)); }
  ~Event() { ember_event_destroy(e_); }
  Event(const Event&) = delete;
  Event& operator=(const Event&) = delete;
  void record() { CTD_CHECK(ember_event_record(e_, runtime::compute_stream())); }
  void wait() { CTD_CHECK(ember_event_synchronize(e_)); }

 private:
  ember_event_t e_ = nullptr;
};

}  // namespace

LoopResult generate_loop(const nn::Model& model, const Request& req,
                         const std::function<void(int64_t)>& emit) {
  using clk = std::chrono::steady_clock;
  const nn::LlamaConfig& cfg = model.config;
  const int prompt_len = static_cast<int>(req.input_ids.size());
  if (prompt_len < 1 || prompt_len >= req.max_seq_len)
    throw std::runtime_error("generate: need 1 <= prompt length < max_seq_len");
  const std::unordered_set<int64_t> eos(req.eos_ids.begin(), req.eos_ids.end());
  nn::KVCache cache = nn::KVCache::allocate(cfg.num_hidden_layers, cfg.num_key_value_heads,
                                            cfg.head_dim, /*batch=*/1, req.max_seq_len, kHIP0);
  ThinkBudget think(req);
  LoopResult res;
  res.reason = "max_tokens";
  const auto t0 = clk::now();
  Tensor prompt =
      Tensor::from_host(req.input_ids.data(), {1, prompt_len}, DType::kInt64, kHIP0);
  Tensor last = model.forward_last_logits(prompt, &cache, 0);

  if (req.sampler.temperature <= 0.0f && !think.active()) {
    // Token t lives in dev[t % 2] and reaches pinned host slot t % 2 through an
    // async copy whose event the host waits on; step t+1 is already queued.
    Tensor dev[2] = {Tensor::empty({1, 1}, DType::kInt64, kHIP0),
                     Tensor::empty({1, 1}, DType::kInt64, kHIP0)};
    Tensor pinned = Tensor::zeros_pinned({2}, DType::kInt64);
    auto* host = static_cast<int64_t*>(pinned.data_ptr());
    Event ready[2];
    auto pick = [&](int slot) {
      device_argmax(last, dev[slot]);
      CTD_CHECK(ember_memcpy_async(host + slot, dev[slot].data_ptr(), sizeof(int64_t), 1,
                                   runtime::compute_stream()));
      ready[slot].record();
    };
    pick(0);
    ready[0].wait();
    res.prefill_ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
    const auto t1 = clk::now();
    for (int t = 0; t < req.max_new_tokens; ++t) {
      const int slot = t % 2;
      const int64_t len = cache.current_len;  // positions before token t's own step
      const bool more = t + 1 < req.max_new_tokens && len + 1 <= req.max_seq_len;
      if (more) {  // token t's step, from the device copy of token t
        last = model.forward_last_logits(dev[slot], &cache, static_cast<int>(len));
        pick(1 - slot);
      }
      ready[slot].wait();
      const int64_t tok = host[slot];
      emit(tok);
      ++res.generated;
      if (eos.count(tok)) {
        res.reason = "eos";
        break;
      }
      if (len + 1 > req.max_seq_len) {
        res.reason = "max_seq_len";
        break;
      }
    }
    runtime::synchronize();  // a speculative step may still be running
    res.decode_ms = std::chrono::duration<double, std::milli>(clk::now() - t1).count();
    return res;
  }

  std::mt19937_64 rng(req.seed);
  runtime::synchronize();
  res.prefill_ms = std::chrono::duration<double, std::milli>(clk::now() - t0).count();
  const auto t1 = clk::now();
  while (res.generated < req.max_new_tokens) {
    int64_t tok;
    if (!think.next_forced(&tok)) tok = sample(last, req.sampler, rng)[0];
    emit(tok);
    ++res.generated;
    think.observe(tok);
    if (eos.count(tok)) {
      res.reason = "eos";
      break;
    }
    if (cache.current_len + 1 > req.max_seq_len) {
      res.reason = "max_seq_len";
      break;
    }
    Tensor next = Tensor::from_host(&tok, {1, 1}, DType::kInt64, kHIP0);
    last = model.forward_last_logits(next, &cache, static_cast<int>(cache.current_len));
  }
  res.decode_ms = std::chrono::duration<double, std::milli>(clk::now() - t1).count();
  return res;
}

int run(const std::string& model_path, const std::string& request, std::ostream& out,
        std::ostream& log, const std::string& model_config) {
  try {
    const Request req = parse_request(request);
    const auto t0 = std::chrono::steady_clock::now();
    log << "ctd_generate: weights " << model_path << "\n";
    const TensorDict weights = load_safetensors(model_path, kHIP0);
    const nn::LlamaConfig cfg = model_config.empty() ? nn::autodetect_config(weights)
                                                     : train::load_model_config(model_config);
    log << "ctd_generate: " << cfg.num_hidden_layers << " layers of width " << cfg.hidden_size
        << ", vocabulary " << cfg.vocab_size << "\n";
    const nn::Model model = nn::build_model(weights, cfg);
    log << "ctd_generate: loaded in " << seconds_since(t0) << " s\n";

    const int prompt_len = static_cast<int>(req.input_ids.size());
    if (prompt_len == 0) {
      out << line(json::ObjectWriter().field("done", true).field("reason", "empty_prompt"))
          << std::flush;
      return 0;
    }
    if (prompt_len >= req.max_seq_len) {
      out << line(json::ObjectWriter().field("done", true).field("reason", "max_seq_len"))
          << std::flush;
      return 0;
    }
    const LoopResult r = generate_loop(model, req, [&](int64_t tok) {
      out << line(json::ObjectWriter().field("token", tok)) << std::flush;
    });
    const double dt = r.decode_ms / 1e3;
    log << "ctd_generate: prompt of " << prompt_len << " tokens in " << r.prefill_ms << " ms, "
        << r.generated << " new tokens in " << dt << " s (" << r.generated / std::max(dt, 1e-9)
        << " tokens/s)\n";
    out << line(json::ObjectWriter()
                    .field("done", true)
                    .field("generated_tokens", r.generated)
                    .field("reason", r.reason))
        << std::flush;
    return 0;
  } catch (const std::exception& e) {
    log << "ctd_generate: error: " << e.what() << "\n";
    out << line(json::ObjectWriter()
                    .field("done", true)
                    .field("error", e.what())
                    .field("reason", "error"))
        << std::flush;
    return 1;
  }
}

}  // namespace ctd::generate
