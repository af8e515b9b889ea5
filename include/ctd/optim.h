#pragma once
// AdamW (decoupled weight decay) with optional host-offloaded m/v, and global
// grad-norm clipping (mirrors include/ctd/optim.h of the reference).
//
//   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2
//   p <- p - lr ( (m/(1-b1^t)) / (sqrt(v/(1-b2^t)) + eps) + wd p )
//
// With offload = true, m and v live in page-locked host memory and step()
// streams them through a ring of device buffers in fixed-size chunks: the
// host->device copies, the fused update on the compute stream and the
// device->host copies of neighbouring chunks overlap on two copy streams.

#include <cstdint>
#include <vector>

#include "ctd/tensor.h"

namespace ctd::optim {

struct ParamGroup {
  std::vector<Tensor> params;
  float lr;
  float weight_decay;
};

struct OffloadStats {
  double last_step_ms = 0.0;       // wall time of the last offloaded step()
  double last_h2d_bytes = 0.0;
  double last_d2h_bytes = 0.0;
};

class AdamW {
 public:
  AdamW(std::vector<Tensor> params, float lr, float weight_decay = 0.0f, float beta1 = 0.9f,
        float beta2 = 0.95f, float eps = 1e-8f, bool offload = false);
  AdamW(std::vector<ParamGroup> groups, float beta1 = 0.9f, float beta2 = 0.95f,
        float eps = 1e-8f, bool offload = false);
  ~AdamW();
  AdamW(const AdamW&) = delete;
  AdamW& operator=(const AdamW&) = delete;

  void step();
  void zero_grad();

  int64_t step_count() const { return step_; }
  bool is_offloaded() const { return offload_; }
  void set_lr(float lr) {
    for (auto& g : groups_) g.lr = lr;
  }
  float lr() const { return groups_.empty() ? 0.0f : groups_.front().lr; }

  void ensure_state_initialized();
  void set_step_count(int64_t s) { step_ = s; }
  size_t num_groups() const { return groups_.size(); }
  size_t num_params(size_t gi) const { return groups_.at(gi).params.size(); }
  Tensor& m_tensor(size_t gi, size_t pi) { return state_.at(gi).at(pi).m; }
  Tensor& v_tensor(size_t gi, size_t pi) { return state_.at(gi).at(pi).v; }

  // Elements per streamed chunk (default 16M floats = 64 MB per buffer).
  // Rounded up to 64 elements so every chunk starts on a 256-byte boundary.
  void set_offload_chunk(int64_t elems) { chunk_elems_ = elems <= 0 ? 64 : (elems + 63) / 64 * 64; }
  const OffloadStats& offload_stats() const { return stats_; }

 private:
  struct State {
    Tensor m;
    Tensor v;
  };

  void init_state_for_group(size_t gi);
  void step_ondevice();
  void step_offloaded();

  std::vector<ParamGroup> groups_;
  std::vector<std::vector<State>> state_;
  float beta1_, beta2_, eps_;
  int64_t step_ = 0;
  bool offload_ = false;

  // Offload ring: kSlots device buffers for m and for v, and the events that
  // order the copy streams against the compute stream.
  static constexpr int kSlots = 3;
  int64_t chunk_elems_ = int64_t{1} << 24;
  float* d_m_[kSlots] = {nullptr, nullptr, nullptr};
  float* d_v_[kSlots] = {nullptr, nullptr, nullptr};
  void* ev_loaded_[kSlots] = {nullptr, nullptr, nullptr};
  void* ev_updated_[kSlots] = {nullptr, nullptr, nullptr};
  void* ev_drained_[kSlots] = {nullptr, nullptr, nullptr};
  void* ev_done_ = nullptr;
  OffloadStats stats_;
};

// Global L2 norm clipping; returns the pre-clip total norm.
float clip_grad_norm_(const std::vector<Tensor>& params, float max_norm, float eps = 1e-6f);

}  // namespace ctd::optim
