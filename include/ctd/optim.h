#pragma once
// SGD, AdamW (decoupled weight decay) with optional host-offloaded m/v, and
// global grad-norm clipping (mirrors include/ctd/optim.h of the reference).
//
//   m = b1 m + (1-b1) g;  v = b2 v + (1-b2) g^2
//   p <- p - lr ( (m/(1-b1^t)) / (sqrt(v/(1-b2^t)) + eps) + wd p )
//
// With offload = true, m and v live in page-locked host memory, one flat
// buffer each with the parameters laid out in streaming order, and step()
// streams them through a ring of device buffers in fixed-size chunks that may
// span several (small) parameters (the first chunks optionally staged ahead of
// step() by prefetch()): the
// host->device copies, the fused update and the device->host copies of
// neighbouring chunks overlap on two copy streams and an optimizer stream.
// step() returns once the work is enqueued; the compute stream is not held
// back by it.  Each parameter's storage carries the event of its own update,
// so the next forward waits only for the parameters it touches, in the order
// it touches them (set_update_order), and the host link stays busy while the
// next step computes.

#include <cstdint>
#include <utility>
#include <vector>

#include "ctd/tensor.h"

namespace ctd::optim {

// Plain SGD, p <- p - lr * g for every parameter with a gradient (the
// reference's include/ctd/optim.h:11-20; it has no momentum or weight decay).
class SGD {
 public:
  explicit SGD(std::vector<Tensor> params, float lr);
  void step();
  void zero_grad();

 private:
  std::vector<Tensor> params_;
  float lr_;
};

struct ParamGroup {
  std::vector<Tensor> params;
  float lr;
  float weight_decay;
};

struct OffloadStats {
  double last_step_ms = 0.0;       // host time to enqueue the last offloaded step()
  double last_h2d_bytes = 0.0;
  double last_d2h_bytes = 0.0;
  // Device time from the first copy in to the last copy out of the most
  // recent offloaded step that has finished (0 until one has).
  double last_stream_ms = 0.0;
  // Bytes per direction (m and v) of the last step's state that prefetch()
  // had copied in before step(); last_h2d_bytes excludes them.
  double last_prefetch_bytes = 0.0;
  // Device time of each direction in the most recent finished step: the
  // copies in from the first to the last (on the h2d stream), the copies out
  // from the first to the last (on the d2h stream, with the updates between
  // them).  Rates per direction are last_h2d_bytes / last_h2d_ms and
  // last_d2h_bytes / last_d2h_ms.
  double last_h2d_ms = 0.0;
  double last_d2h_ms = 0.0;
  // Bytes per direction the last step did not move because no parameter in
  // them had a gradient (frozen or unused parameters keep their m/v on the host).
  double last_skipped_bytes = 0.0;
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
  // Optimizer state; with offload these are host tensors that an in-flight
  // step() still writes, so both accessors first wait for it to finish, and
  // they drop a pending prefetch() (the caller may change the state it copied).
  Tensor& m_tensor(size_t gi, size_t pi);
  Tensor& v_tensor(size_t gi, size_t pi);

  // Elements per streamed chunk (default 16M floats = 64 MB per buffer).
  // Rounded up to 64 elements so every chunk starts on a 256-byte boundary.
  void set_offload_chunk(int64_t elems) { chunk_elems_ = elems <= 0 ? 64 : (elems + 63) / 64 * 64; }
  // Order in which the offloaded step streams parameters, as (group, index)
  // pairs; parameters not listed follow in group order.  Give the order in
  // which the forward pass first reads them, so it can start on the first
  // parameters while the rest are still in flight.  It fixes the host layout
  // of m and v, so it must come before the state exists (first step(),
  // ensure_state_initialized()).
  void set_update_order(std::vector<std::pair<size_t, size_t>> order);
  // Stages on the device the optimizer state of the first parameters in
  // streaming order -- the chunks that cover the first parameter, at most
  // set_prefetch_chunks() of them -- copying it in on the h2d stream once the
  // compute stream has reached this call.  The next step() updates those
  // chunks as soon as the gradients are final instead of after their
  // transfer, so the next forward, which reads that parameter first, waits
  // for less; it hands the buffer back once they are copied out.  Meant for
  // late in the backward pass, when the host link is idle and most
  // activations are freed.  Does nothing without offload, with a prefetch
  // already pending, or with set_prefetch_chunks(0).
  void prefetch();
  void set_prefetch_chunks(int64_t n) { max_prefetch_chunks_ = n < 0 ? 0 : n; }
  // Blocks until the last offloaded step() has finished on every stream.
  void wait_idle();
  const OffloadStats& offload_stats();

 private:
  struct State {
    Tensor m;
    Tensor v;
  };

  // One parameter's place in the flat offloaded state (streaming order).
  struct Segment {
    size_t gi, pi;
    int64_t off, n;
  };

  void init_state_for_group(size_t gi);
  void init_offload_state();
  void step_ondevice();
  void step_offloaded();
  void drop_prefetch();  // wait for a pending prefetch's copies and discard them

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
  void* ev_begin_ = nullptr;   // on the h2d stream before the first copy in
  void* ev_start_ = nullptr;   // on the compute stream: grads and params final
  bool in_flight_ = false;     // an offloaded step was enqueued and not yet waited on
  std::vector<std::vector<void*>> ev_param_;  // per parameter: its update is done
  std::vector<std::pair<size_t, size_t>> order_;
  std::vector<Segment> layout_;  // offloaded state, in streaming order
  Tensor flat_m_, flat_v_;       // pinned host buffers the per-parameter m/v view
  int64_t flat_n_ = 0;
  OffloadStats stats_;
  // prefetch(): device copies of the state's first pf_elems_ floats, made with
  // chunks of pf_chunk_elems_ (0 elements: nothing pending).
  int64_t max_prefetch_chunks_ = 32;
  Tensor pf_m_, pf_v_;
  int64_t pf_elems_ = 0, pf_chunk_elems_ = 0;
  void* ev_pf_ready_ = nullptr;    // compute stream: the buffer's memory is free
  void* ev_pf_loaded_ = nullptr;   // h2d stream: the prefetch copies are done
  void* ev_pf_drained_ = nullptr;  // d2h stream: its chunks are copied out
  void* ev_h2d_end_ = nullptr;     // h2d stream: after the step's last copy in
  void* ev_d2h_begin_ = nullptr;   // d2h stream: before the step's first copy out
};

// Global L2 norm clipping; returns the pre-clip total norm.
float clip_grad_norm_(const std::vector<Tensor>& params, float max_norm, float eps = 1e-6f);

}  // namespace ctd::optim
