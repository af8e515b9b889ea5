#pragma once
// Token generation behind the ctd_generate stdin/stdout protocol (reference
// tools/ctd_generate/main.cpp:52-192).
//
// Request: one JSON object,
//   {"input_ids": [int...],            required
//    "max_new_tokens": 64, "max_seq_len": 2048,
//    "temperature": 1.0, "top_k": 0, "top_p": 0.0, "seed": 0,
//    "eos_ids": [int...],
//    "thinking_token_budget": 0, "think_open_ids": [...], "think_close_ids": [...]}
// Reply: one JSON line per generated token {"token":id}, then
//   {"done":true,"generated_tokens":n,"reason":"max_tokens"|"eos"|"max_seq_len"},
// or {"done":true,"reason":"empty_prompt"|"max_seq_len"} before any token, or
// {"done":true,"error":"...","reason":"error"} on failure.  Keys are sorted.
#include <cstdint>
#include <functional>
#include <ostream>
#include <string>
#include <vector>

#include "ctd/nn/model.h"
#include "ctd/sampling.h"

namespace ctd::generate {

struct Request {
  std::vector<int64_t> input_ids;
  int max_new_tokens = 64;
  int max_seq_len = 2048;
  SamplerConfig sampler;
  uint64_t seed = 0;
  std::vector<int64_t> eos_ids;
  int thinking_token_budget = 0;
  std::vector<int64_t> think_open_ids;
  std::vector<int64_t> think_close_ids;
};

// Parses a request; throws std::runtime_error on bad JSON or field types.
Request parse_request(const std::string& text);

// Budget forcing (main.cpp:88-98, 133-171): once a thinking span (opened by
// think_open_ids) has run thinking_token_budget tokens, think_close_ids are
// emitted next instead of sampled tokens.
class ThinkBudget {
 public:
  ThinkBudget(const Request& r);
  bool active() const { return active_; }
  // A forced token to emit now, if any (pops it).
  bool next_forced(int64_t* tok);
  // Records an emitted token.
  void observe(int64_t tok);

 private:
  bool ends_with(const std::vector<int64_t>& seq) const;
  bool active_ = false;
  int budget_ = 0;
  std::vector<int64_t> open_, close_;
  std::vector<int64_t> window_, queue_;
  size_t cap_ = 0;
  bool in_think_ = false;
  int count_ = 0;
};

struct LoopResult {
  int generated = 0;
  std::string reason;       // "max_tokens", "eos" or "max_seq_len"
  double prefill_ms = 0.0;  // host wall time: prompt in, first logits ready
  double decode_ms = 0.0;   // host wall time of the token loop
};

// The generation loop of run() over a built model, batch 1: prefill the
// prompt (req.input_ids non-empty, shorter than req.max_seq_len), then up to
// max_new_tokens tokens, calling emit(token) for each in order.  Greedy
// requests without budget forcing keep the token on the device: step t+1 is
// enqueued before the host reads token t, which only decides whether to stop.
LoopResult generate_loop(const nn::Model& model, const Request& req,
                         const std::function<void(int64_t)>& emit);

// Runs the protocol for one request text with the model at model_path:
// writes the JSON reply lines to out and progress to log.  Returns the exit
// status (0, or 1 after an error line).  The architecture is detected from the
// embedding shape (nn::autodetect_config) unless model_config names a JSON
// file with the fields of ctd_train's "model" object.
int run(const std::string& model_path, const std::string& request, std::ostream& out,
        std::ostream& log, const std::string& model_config = "");

}  // namespace ctd::generate
