// AdamW (on-device and host-offloaded) and global grad-norm clipping.
//
// Reference: src/core/optim.cu:77-293.  The offloaded path there keeps m/v in
// pageable host memory and runs, per parameter, two synchronous H2D copies,
// the kernel and two synchronous D2H copies (optim.cu:176-210).  Here m/v are
// page-locked, every parameter is cut into chunks of chunk_elems_ floats, and
// chunk i flows through a ring of kSlots device buffers:
//
//   h2d stream:     wait drained[s] -> copy m,v chunk i in  -> record loaded[s]
//   compute stream: wait loaded[s]  -> AdamW on chunk i      -> record updated[s]
//   d2h stream:     wait updated[s] -> copy m,v chunk i out -> record drained[s]
//
// with s = i % kSlots, so the copies in of chunk i+1, the update of chunk i
// and the copies out of chunk i-1 run at the same time, and both link
// directions stay busy.  The compute stream finally waits for the last copy
// out, so anything ordered after step() sees the finished state.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <stdexcept>

#include "ctd/optim.h"
#include "op_util.h"

namespace ctd::optim {

using namespace ctd::ops::detail;

AdamW::AdamW(std::vector<Tensor> params, float lr, float weight_decay, float beta1, float beta2,
             float eps, bool offload)
    : AdamW(std::vector<ParamGroup>{ParamGroup{std::move(params), lr, weight_decay}}, beta1, beta2,
            eps, offload) {}

AdamW::AdamW(std::vector<ParamGroup> groups, float beta1, float beta2, float eps, bool offload)
    : groups_(std::move(groups)), beta1_(beta1), beta2_(beta2), eps_(eps), offload_(offload) {
  state_.resize(groups_.size());
  for (const auto& g : groups_)
    for (const auto& p : g.params) {
      if (!p.requires_grad()) throw std::runtime_error("AdamW: param does not require grad");
      if (p.dtype() != DType::kFloat32) throw std::runtime_error("AdamW: fp32 only");
      if (!p.device().is_hip()) throw std::runtime_error("AdamW: params must be on the HIP device");
    }
}

AdamW::~AdamW() {
  if (ev_done_) ember_event_synchronize(ev_done_);
  for (int s = 0; s < kSlots; ++s) {
    ember_device_free(d_m_[s]);
    ember_device_free(d_v_[s]);
    ember_event_destroy(ev_loaded_[s]);
    ember_event_destroy(ev_updated_[s]);
    ember_event_destroy(ev_drained_[s]);
  }
  ember_event_destroy(ev_done_);
}

void AdamW::ensure_state_initialized() {
  for (size_t gi = 0; gi < groups_.size(); ++gi) init_state_for_group(gi);
}

void AdamW::init_state_for_group(size_t gi) {
  auto& g = groups_[gi];
  auto& st = state_[gi];
  if (st.size() == g.params.size()) return;
  st.clear();
  st.reserve(g.params.size());
  int64_t largest = 0;
  for (const auto& p : g.params) {
    State s;
    if (offload_) {
      s.m = Tensor::zeros_pinned(p.shape(), p.dtype());
      s.v = Tensor::zeros_pinned(p.shape(), p.dtype());
    } else {
      s.m = Tensor::zeros(p.shape(), p.dtype(), p.device());
      s.v = Tensor::zeros(p.shape(), p.dtype(), p.device());
    }
    largest = std::max(largest, p.numel());
    st.push_back(std::move(s));
  }
  if (offload_ && !d_m_[0]) {
    // Slots never need to be larger than the largest parameter of the group.
    chunk_elems_ = std::max<int64_t>(1, std::min(chunk_elems_, largest));
    for (int s = 0; s < kSlots; ++s) {
      void* pm = nullptr;
      void* pv = nullptr;
      CTD_CHECK(ember_device_malloc(&pm, static_cast<size_t>(chunk_elems_) * sizeof(float)));
      CTD_CHECK(ember_device_malloc(&pv, static_cast<size_t>(chunk_elems_) * sizeof(float)));
      d_m_[s] = static_cast<float*>(pm);
      d_v_[s] = static_cast<float*>(pv);
      CTD_CHECK(ember_event_create(&ev_loaded_[s]));
      CTD_CHECK(ember_event_create(&ev_updated_[s]));
      CTD_CHECK(ember_event_create(&ev_drained_[s]));
    }
    CTD_CHECK(ember_event_create(&ev_done_));
  }
}

void AdamW::step() {
  ++step_;
  if (offload_)
    step_offloaded();
  else
    step_ondevice();
}

void AdamW::step_ondevice() {
  // Bias corrections in host float (optim.cu:142-143).
  const float bc1 = 1.0f - std::pow(beta1_, static_cast<float>(step_));
  const float bc2 = 1.0f - std::pow(beta2_, static_cast<float>(step_));
  for (size_t gi = 0; gi < groups_.size(); ++gi) {
    init_state_for_group(gi);
    auto& group = groups_[gi];
    auto& st = state_[gi];
    for (size_t pi = 0; pi < group.params.size(); ++pi) {
      Tensor& p = group.params[pi];
      Tensor g = p.grad();
      if (!g.storage()) continue;
      if (g.shape() != p.shape()) throw std::runtime_error("AdamW: param/grad shape mismatch");
      CTD_CHECK(ember_adamw(fp(p), cfp(g), fp(st[pi].m), fp(st[pi].v), p.numel(), group.lr, beta1_,
                            beta2_, eps_, group.weight_decay, bc1, bc2, S()));
    }
  }
}

void AdamW::step_offloaded() {
  const auto t0 = std::chrono::steady_clock::now();
  const float bc1 = 1.0f - std::pow(beta1_, static_cast<float>(step_));
  const float bc2 = 1.0f - std::pow(beta2_, static_cast<float>(step_));
  for (size_t gi = 0; gi < groups_.size(); ++gi) init_state_for_group(gi);
  ember_stream_t cs = S(), hs = runtime::h2d_stream(), ds = runtime::d2h_stream();

  // Grads and params are produced on the compute stream; the copy streams only
  // touch the pinned host state and the ring buffers, so they need no wait for
  // the backward pass.  The previous step's last copy out must be finished
  // before this step overwrites the same host buffers' device copies.
  if (step_ > 1) CTD_CHECK(ember_stream_wait_event(hs, ev_done_));

  int64_t chunk = 0;
  double bytes = 0.0;
  for (size_t gi = 0; gi < groups_.size(); ++gi) {
    auto& group = groups_[gi];
    auto& st = state_[gi];
    for (size_t pi = 0; pi < group.params.size(); ++pi) {
      Tensor& p = group.params[pi];
      Tensor g = p.grad();
      if (!g.storage()) continue;
      if (g.shape() != p.shape()) throw std::runtime_error("AdamW: param/grad shape mismatch");
      float* hm = static_cast<float*>(st[pi].m.data_ptr());
      float* hv = static_cast<float*>(st[pi].v.data_ptr());
      const int64_t n = p.numel();
      for (int64_t off = 0; off < n; off += chunk_elems_, ++chunk) {
        const int64_t len = std::min(chunk_elems_, n - off);
        const size_t nb = static_cast<size_t>(len) * sizeof(float);
        const int s = static_cast<int>(chunk % kSlots);
        if (chunk >= kSlots) CTD_CHECK(ember_stream_wait_event(hs, ev_drained_[s]));
        CTD_CHECK(ember_memcpy_async(d_m_[s], hm + off, nb, 0, hs));
        CTD_CHECK(ember_memcpy_async(d_v_[s], hv + off, nb, 0, hs));
        CTD_CHECK(ember_event_record(ev_loaded_[s], hs));
        CTD_CHECK(ember_stream_wait_event(cs, ev_loaded_[s]));
        CTD_CHECK(ember_adamw(fp(p) + off, cfp(g) + off, d_m_[s], d_v_[s], len, group.lr, beta1_,
                              beta2_, eps_, group.weight_decay, bc1, bc2, cs));
        CTD_CHECK(ember_event_record(ev_updated_[s], cs));
        CTD_CHECK(ember_stream_wait_event(ds, ev_updated_[s]));
        CTD_CHECK(ember_memcpy_async(hm + off, d_m_[s], nb, 1, ds));
        CTD_CHECK(ember_memcpy_async(hv + off, d_v_[s], nb, 1, ds));
        CTD_CHECK(ember_event_record(ev_drained_[s], ds));
        bytes += 2.0 * static_cast<double>(nb);
      }
    }
  }
  CTD_CHECK(ember_event_record(ev_done_, ds));
  CTD_CHECK(ember_stream_wait_event(cs, ev_done_));
  stats_.last_h2d_bytes = bytes;
  stats_.last_d2h_bytes = bytes;
  stats_.last_step_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

void AdamW::zero_grad() {
  for (auto& g : groups_)
    for (auto& p : g.params) p.zero_grad_();
}

float clip_grad_norm_(const std::vector<Tensor>& params, float max_norm, float eps) {
  std::vector<const float*> ptrs;
  std::vector<int64_t> sizes;
  std::vector<Tensor> grads;
  for (const auto& p : params) {
    Tensor g = p.grad();
    if (!g.storage()) continue;
    if (p.dtype() != DType::kFloat32) throw std::runtime_error("clip_grad_norm_: fp32 only");
    if (g.numel() == 0) continue;
    ptrs.push_back(cfp(g));
    sizes.push_back(g.numel());
    grads.push_back(g);
  }
  const int count = static_cast<int>(ptrs.size());
  const size_t wsb = ember_sumsq_workspace_bytes(count);
  Tensor ws = wsb ? workspace(wsb) : Tensor{};
  Tensor out = Tensor::empty({1}, DType::kFloat32, kHIP0);
  CTD_CHECK(ember_sumsq_multi(ptrs.data(), sizes.data(), count, fp(out),
                              wsb ? ws.data_ptr() : nullptr, wsb, S()));
  float sum = 0.0f;
  out.copy_to_host(&sum);
  const float total = std::sqrt(sum);
  if (total > max_norm) {
    const float scale = max_norm / (total + eps);
    for (auto& g : grads) CTD_CHECK(ember_scale(cfp(g), scale, fp(g), g.numel(), S()));
  }
  return total;
}

}  // namespace ctd::optim
