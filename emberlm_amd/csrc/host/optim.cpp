// AdamW (on-device and host-offloaded) and global grad-norm clipping.
//
// Reference: src/core/optim.cu:77-293.  The offloaded path there keeps m/v in
// pageable host memory and runs, per parameter, two synchronous H2D copies,
// the kernel and two synchronous D2H copies (optim.cu:176-210).  Here m/v are
// page-locked and laid out as one flat buffer each, parameters back to back in
// streaming order (each starting on a 256-byte boundary), and the buffer is
// cut into chunks of chunk_elems_ floats that may span several parameters --
// a per-parameter cut would send hundreds of tiny norm-weight transfers,
// whose fixed cost halves the link rate.  Chunk i flows through a ring of
// kSlots device buffers:
//
//   h2d stream: wait drained[s] -> copy m,v chunk i in -> record loaded[s]
//   d2h stream: wait loaded[s]  -> AdamW on each parameter piece of chunk i
//               -> copy m,v chunk i out -> record drained[s]
//
// with s = i % kSlots, so the copies in of chunks i+1.. run while chunk i is
// updated and copied out, and both link directions stay busy.  The update
// kernels start after everything the compute stream has enqueued so far
// (backward, clipping).  The compute
// stream is not made to wait for the whole step: each parameter's storage
// (and its gradient's) gets the event recorded after its last chunk's update,
// and the first data_ptr() of that storage makes the compute stream wait for
// exactly that event.  The next forward therefore starts as soon as its first
// parameters are updated and the remaining transfers hide behind it.  Each
// gradient stays alive until its parameter's update has run (release_after),
// since zero_grad() lets go of it while the update may still be reading it.
//
// The forward reads the first parameter in streaming order (the embedding)
// first, and waits for its update.  prefetch(), called late in the backward
// while the host link is idle, copies the chunks covering that parameter into
// a device buffer from the caching allocator; step() then runs their updates
// before any copy, so that parameter is final a few kernels after the
// backward ends, and copies them out after the ring.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <stdexcept>

#include "ctd/optim.h"
#include "op_util.h"

namespace ctd::optim {

using namespace ctd::ops::detail;

namespace {
// Workgroups of one chunk update: four per CU, of the 22-register scalar
// form, so they fit next to the forward's GEMM and attention blocks.  The
// update runs on the d2h stream between a chunk's arrival and its copy out,
// so its length adds to the link's idle time: one workgroup per CU (one load
// in flight per lane) took 307 ms for the isolated offloaded step of a
// 1.7B-parameter model, four per CU 297 ms, the same as four times the loads
// in flight per lane (unrolled or float4) at one or two per CU.
constexpr int kUpdateBlocks = 1024;
}  // namespace

// ------------------------------------------------------------------ SGD
// src/core/optim.cu:23-48 of the reference: every parameter must require grad;
// step() updates those that have a gradient, one launch each.
SGD::SGD(std::vector<Tensor> params, float lr) : params_(std::move(params)), lr_(lr) {
  for (const Tensor& p : params_)
    if (!p.requires_grad()) throw std::runtime_error("SGD: param does not require grad");
}

void SGD::step() {
  for (Tensor& p : params_) {
    Tensor g = p.grad();
    if (!g.storage()) continue;
    if (g.shape() != p.shape()) throw std::runtime_error("SGD: param/grad shape mismatch");
    if (p.dtype() != DType::kFloat32 || g.dtype() != DType::kFloat32)
      throw std::runtime_error("SGD: fp32 only");
    CTD_CHECK(ember_sgd(static_cast<float*>(p.data_ptr()), static_cast<const float*>(g.data_ptr()),
                        p.numel(), lr_, runtime::compute_stream()));
  }
}

void SGD::zero_grad() {
  for (Tensor& p : params_) p.zero_grad_();
}

// ---------------------------------------------------------------- AdamW
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
  if (in_flight_ && ev_done_) ember_event_synchronize(ev_done_);
  // A pending prefetch's copies must land before its buffer goes back to the
  // allocator (no throwing from a destructor: the status is not checked).
  if (pf_elems_ > 0 && ev_pf_loaded_) ember_event_synchronize(ev_pf_loaded_);
  pf_m_ = Tensor{};
  pf_v_ = Tensor{};
  runtime::collect_released();
  // Our events die with us: no storage may keep pointing at them.
  for (size_t gi = 0; gi < ev_param_.size(); ++gi)
    for (size_t pi = 0; pi < ev_param_[gi].size(); ++pi) {
      Tensor& p = groups_[gi].params[pi];
      if (p.storage() && p.storage()->ready_event() == ev_param_[gi][pi])
        p.storage()->set_ready_event(nullptr);
      Tensor g = p.grad();
      if (g.storage() && g.storage()->ready_event() == ev_param_[gi][pi])
        g.storage()->set_ready_event(nullptr);
      ember_event_destroy(ev_param_[gi][pi]);
    }
  for (int s = 0; s < kSlots; ++s) {
    ember_device_free(d_m_[s]);
    ember_device_free(d_v_[s]);
    ember_event_destroy(ev_loaded_[s]);
    ember_event_destroy(ev_updated_[s]);
    ember_event_destroy(ev_drained_[s]);
  }
  ember_event_destroy(ev_done_);
  ember_event_destroy(ev_begin_);
  ember_event_destroy(ev_start_);
  ember_event_destroy(ev_pf_ready_);
  ember_event_destroy(ev_pf_loaded_);
  ember_event_destroy(ev_pf_drained_);
  ember_event_destroy(ev_h2d_end_);
  ember_event_destroy(ev_d2h_begin_);
}

Tensor& AdamW::m_tensor(size_t gi, size_t pi) {
  wait_idle();
  drop_prefetch();  // the caller may write the host state the prefetch copied
  return state_.at(gi).at(pi).m;
}

Tensor& AdamW::v_tensor(size_t gi, size_t pi) {
  wait_idle();
  drop_prefetch();
  return state_.at(gi).at(pi).v;
}

void AdamW::drop_prefetch() {
  if (pf_elems_ <= 0) return;
  CTD_CHECK(ember_event_synchronize(ev_pf_loaded_));
  pf_m_ = Tensor{};
  pf_v_ = Tensor{};
  pf_elems_ = 0;
}

void AdamW::set_update_order(std::vector<std::pair<size_t, size_t>> order) {
  for (const auto& [gi, pi] : order)
    if (gi >= groups_.size() || pi >= groups_[gi].params.size())
      throw std::runtime_error("AdamW::set_update_order: index out of range");
  if (!layout_.empty() && order != order_)
    throw std::runtime_error("AdamW::set_update_order: optimizer state already laid out");
  order_ = std::move(order);
}

void AdamW::wait_idle() {
  if (in_flight_) {
    CTD_CHECK(ember_event_synchronize(ev_done_));
    float ms = 0.f;
    CTD_CHECK(ember_event_elapsed_ms(&ms, ev_begin_, ev_done_));
    stats_.last_stream_ms = ms;
    CTD_CHECK(ember_event_elapsed_ms(&ms, ev_begin_, ev_h2d_end_));
    stats_.last_h2d_ms = ms;
    CTD_CHECK(ember_event_elapsed_ms(&ms, ev_d2h_begin_, ev_done_));
    stats_.last_d2h_ms = ms;
    in_flight_ = false;
  }
  runtime::collect_released();
}

const OffloadStats& AdamW::offload_stats() { return stats_; }

void AdamW::ensure_state_initialized() {
  if (offload_) {
    init_offload_state();
    return;
  }
  for (size_t gi = 0; gi < groups_.size(); ++gi) init_state_for_group(gi);
}

void AdamW::init_state_for_group(size_t gi) {
  auto& g = groups_[gi];
  auto& st = state_[gi];
  if (st.size() == g.params.size()) return;
  st.clear();
  st.reserve(g.params.size());
  for (const auto& p : g.params) {
    State s;
    s.m = Tensor::zeros(p.shape(), p.dtype(), p.device());
    s.v = Tensor::zeros(p.shape(), p.dtype(), p.device());
    st.push_back(std::move(s));
  }
}

void AdamW::init_offload_state() {
  if (!layout_.empty() || groups_.empty()) return;
  // Streaming order: the requested one, then whatever it left out.
  std::vector<std::vector<bool>> seen(groups_.size());
  for (size_t gi = 0; gi < groups_.size(); ++gi) seen[gi].assign(groups_[gi].params.size(), false);
  std::vector<std::pair<size_t, size_t>> items;
  for (const auto& it : order_)
    if (!seen[it.first][it.second]) {
      seen[it.first][it.second] = true;
      items.push_back(it);
    }
  for (size_t gi = 0; gi < groups_.size(); ++gi)
    for (size_t pi = 0; pi < groups_[gi].params.size(); ++pi)
      if (!seen[gi][pi]) items.emplace_back(gi, pi);
  int64_t off = 0;
  for (const auto& [gi, pi] : items) {
    const int64_t n = groups_[gi].params[pi].numel();
    layout_.push_back({gi, pi, off, n});
    off += (n + 63) / 64 * 64;
  }
  flat_n_ = off;
  flat_m_ = Tensor::zeros_pinned({std::max<int64_t>(flat_n_, 1)}, DType::kFloat32);
  flat_v_ = Tensor::zeros_pinned({std::max<int64_t>(flat_n_, 1)}, DType::kFloat32);
  for (size_t gi = 0; gi < groups_.size(); ++gi) state_[gi].assign(groups_[gi].params.size(), {});
  for (const auto& sg : layout_) {
    const Tensor& p = groups_[sg.gi].params[sg.pi];
    state_[sg.gi][sg.pi].m = flat_m_.view_at(sg.off, p.shape());
    state_[sg.gi][sg.pi].v = flat_v_.view_at(sg.off, p.shape());
  }
  if (!d_m_[0]) {
    // Slots never need to be larger than the whole state.
    chunk_elems_ = std::max<int64_t>(64, std::min(chunk_elems_, flat_n_));
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
    CTD_CHECK(ember_event_create(&ev_begin_));
    CTD_CHECK(ember_event_create(&ev_start_));
    CTD_CHECK(ember_event_create(&ev_pf_ready_));
    CTD_CHECK(ember_event_create(&ev_pf_loaded_));
    CTD_CHECK(ember_event_create(&ev_pf_drained_));
    CTD_CHECK(ember_event_create(&ev_h2d_end_));
    CTD_CHECK(ember_event_create(&ev_d2h_begin_));
  }
  ev_param_.resize(groups_.size());
  for (size_t gi = 0; gi < groups_.size(); ++gi)
    while (ev_param_[gi].size() < groups_[gi].params.size()) {
      void* e = nullptr;
      CTD_CHECK(ember_event_create(&e));
      ev_param_[gi].push_back(e);
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

void AdamW::prefetch() {
  if (!offload_ || max_prefetch_chunks_ <= 0 || pf_elems_ > 0) return;
  init_offload_state();
  if (layout_.empty() || flat_n_ <= 0) return;
  const Segment& first = layout_.front();
  const int64_t nch = std::min((first.off + first.n + chunk_elems_ - 1) / chunk_elems_,
                               max_prefetch_chunks_);
  int64_t elems = std::min(nch * chunk_elems_, flat_n_);
  // Fewer chunks when the allocator's largest free block holds fewer (at
  // least one): the staging then fills a hole instead of growing the memory
  // held, and the step streams the rest through the ring as usual.
  const auto fit = [&](int64_t want) {
    const size_t got = elastic_workspace_bytes(static_cast<size_t>(want) * sizeof(float),
                                               static_cast<size_t>(chunk_elems_) * sizeof(float));
    const int64_t n = static_cast<int64_t>(got / sizeof(float));
    return n >= want ? want : std::max<int64_t>(chunk_elems_, n / chunk_elems_ * chunk_elems_);
  };
  elems = std::min(elems, fit(elems));
  ember_stream_t cs = S(), hs = runtime::h2d_stream();
  // The buffer comes from the caching allocator, which orders reuse on the
  // compute stream: the copies wait until that stream has reached this call.
  // They also wait for the previous step's copies out, which write the host
  // state read here.
  pf_m_ = Tensor::empty({elems}, DType::kFloat32, kHIP0);
  if (const int64_t v_elems = fit(elems); v_elems < elems) {
    elems = v_elems;
    pf_m_ = Tensor{};
    pf_m_ = Tensor::empty({elems}, DType::kFloat32, kHIP0);
  }
  pf_v_ = Tensor::empty({elems}, DType::kFloat32, kHIP0);
  CTD_CHECK(ember_event_record(ev_pf_ready_, cs));
  CTD_CHECK(ember_stream_wait_event(hs, ev_pf_ready_));
  if (in_flight_) CTD_CHECK(ember_stream_wait_event(hs, ev_done_));
  const size_t nb = static_cast<size_t>(elems) * sizeof(float);
  CTD_CHECK(ember_memcpy_async(pf_m_.data_ptr(), flat_m_.data_ptr(), nb, 0, hs));
  CTD_CHECK(ember_memcpy_async(pf_v_.data_ptr(), flat_v_.data_ptr(), nb, 0, hs));
  CTD_CHECK(ember_event_record(ev_pf_loaded_, hs));
  pf_elems_ = elems;
  pf_chunk_elems_ = chunk_elems_;
}

void AdamW::step_offloaded() {
  const auto t0 = std::chrono::steady_clock::now();
  const float bc1 = 1.0f - std::pow(beta1_, static_cast<float>(step_));
  const float bc2 = 1.0f - std::pow(beta2_, static_cast<float>(step_));
  init_offload_state();
  // The previous step has long finished by now (the forward and backward in
  // between waited for every parameter it updated); this also frees its ring
  // slots and hands back the gradients it kept.
  wait_idle();
  // The update kernels share the d2h stream: each chunk's kernels then its
  // copies out, in order.  A separate kernel stream would cost one more
  // hardware queue, and with more streams than queues the runtime makes
  // streams share queues, which serialises them against the compute stream.
  ember_stream_t cs = S(), hs = runtime::h2d_stream(), ds = runtime::d2h_stream();
  CTD_CHECK(ember_event_record(ev_start_, cs));
  CTD_CHECK(ember_stream_wait_event(ds, ev_start_));
  CTD_CHECK(ember_event_record(ev_begin_, hs));
  // A prefetch cut with another chunk size does not line up with this
  // step's chunks: let it land and drop it.
  if (pf_chunk_elems_ != chunk_elems_) drop_prefetch();
  const int64_t pf_elems = pf_elems_;
  float* pf_m = pf_elems > 0 ? static_cast<float*>(pf_m_.data_ptr()) : nullptr;
  float* pf_v = pf_elems > 0 ? static_cast<float*>(pf_v_.data_ptr()) : nullptr;
  // The ring's copies are submitted only once the prefetch's have landed.
  // Submitted while those still ran, the copies in and out of the whole step
  // went one after the other instead of both directions at once (measured on
  // MI355X: 333 instead of 215 ms at LLaMA-3.2-1B's 9.9 GB per direction),
  // so the host waits here for whatever part of the prefetch is left.
  if (pf_elems > 0) CTD_CHECK(ember_event_synchronize(ev_pf_loaded_));

  // Device pointers of every parameter with a gradient, in layout order
  // (taken before any storage gets this step's ready event).
  struct Work {
    float* p = nullptr;
    const float* g = nullptr;
  };
  std::vector<Work> work(layout_.size());
  for (size_t k = 0; k < layout_.size(); ++k) {
    const Segment& sg = layout_[k];
    Tensor& p = groups_[sg.gi].params[sg.pi];
    Tensor g = p.grad();
    if (!g.storage()) continue;
    if (g.shape() != p.shape()) throw std::runtime_error("AdamW: param/grad shape mismatch");
    work[k] = {fp(p), cfp(g)};
  }

  float* hm = static_cast<float*>(flat_m_.data_ptr());
  float* hv = static_cast<float*>(flat_v_.data_ptr());
  size_t k = 0;  // first segment not yet finished
  // Updates every parameter piece with a gradient inside [c0, c0 + len),
  // whose m/v sit on the device at cm/cv from state element `base` on, and
  // marks each parameter that ends there as done.
  auto update_range = [&](int64_t c0, int64_t len, int64_t base, float* cm, float* cv) {
    while (k < layout_.size() && layout_[k].off < c0 + len) {
      const Segment& sg = layout_[k];
      const int64_t lo = std::max(sg.off, c0), hi = std::min(sg.off + sg.n, c0 + len);
      if (work[k].p && hi > lo) {
        const ParamGroup& group = groups_[sg.gi];
        CTD_CHECK(ember_adamw_bounded(work[k].p + (lo - sg.off), work[k].g + (lo - sg.off),
                                      cm + (lo - base), cv + (lo - base), hi - lo, group.lr,
                                      beta1_, beta2_, eps_, group.weight_decay, bc1, bc2,
                                      kUpdateBlocks, ds));
      }
      if (sg.off + sg.n > c0 + len) break;  // continues in the next chunk
      if (work[k].p) {
        CTD_CHECK(ember_event_record(ev_param_[sg.gi][sg.pi], ds));
        // The gradient is dead once its update has run: hand its block back
        // then, not at the end of the step, so the next forward does not
        // carry it.
        runtime::release_after(ev_param_[sg.gi][sg.pi],
                               {groups_[sg.gi].params[sg.pi].grad().storage()});
      }
      ++k;
    }
  };

  // [lo, hi) of the state in [c0, c0 + len) that belongs to parameters with
  // a gradient (empty when none has one): only that part crosses the link.
  auto graded_span = [&](int64_t c0, int64_t len) {
    int64_t lo = c0 + len, hi = c0;
    for (size_t j = k; j < layout_.size() && layout_[j].off < c0 + len; ++j) {
      const Segment& sg = layout_[j];
      if (!work[j].p || sg.off + sg.n <= c0) continue;
      lo = std::min(lo, std::max(sg.off, c0));
      hi = std::max(hi, std::min(sg.off + sg.n, c0 + len));
    }
    return std::pair<int64_t, int64_t>{lo, hi};
  };

  double bytes_in = 0.0, bytes_out = 0.0, skipped = 0.0;
  bool first_out = true;
  auto mark_first_out = [&] {
    if (first_out) CTD_CHECK(ember_event_record(ev_d2h_begin_, ds));
    first_out = false;
  };
  // The prefetched state (a whole number of chunks, or the whole state) is
  // updated before anything else and copied out after everything else: the
  // d2h stream runs the updates in streaming order, which is the order the
  // next forward waits for them, and no copy of it holds back a later one.
  if (pf_elems > 0) update_range(0, pf_elems, 0, pf_m, pf_v);
  int64_t ring = 0;  // chunks streamed through the ring so far
  for (int64_t c0 = pf_elems; c0 < flat_n_; c0 += chunk_elems_) {
    const int64_t len = std::min(chunk_elems_, flat_n_ - c0);
    const auto [lo, hi] = graded_span(c0, len);
    skipped += 2.0 * static_cast<double>(len - std::max<int64_t>(hi - lo, 0)) * sizeof(float);
    if (hi <= lo) {  // no gradient in this chunk: its state stays on the host
      update_range(c0, len, c0, nullptr, nullptr);
      continue;
    }
    const size_t nb = static_cast<size_t>(hi - lo) * sizeof(float);
    const int s = static_cast<int>(ring % kSlots);
    if (ring >= kSlots) CTD_CHECK(ember_stream_wait_event(hs, ev_drained_[s]));
    CTD_CHECK(ember_memcpy_async(d_m_[s], hm + lo, nb, 0, hs));
    CTD_CHECK(ember_memcpy_async(d_v_[s], hv + lo, nb, 0, hs));
    CTD_CHECK(ember_event_record(ev_loaded_[s], hs));
    CTD_CHECK(ember_stream_wait_event(ds, ev_loaded_[s]));
    update_range(c0, len, lo, d_m_[s], d_v_[s]);  // the slot holds [lo, hi)
    mark_first_out();
    CTD_CHECK(ember_memcpy_async(hm + lo, d_m_[s], nb, 1, ds));
    CTD_CHECK(ember_memcpy_async(hv + lo, d_v_[s], nb, 1, ds));
    CTD_CHECK(ember_event_record(ev_drained_[s], ds));
    bytes_in += 2.0 * static_cast<double>(nb);
    bytes_out += 2.0 * static_cast<double>(nb);
    ++ring;
  }
  CTD_CHECK(ember_event_record(ev_h2d_end_, hs));
  if (pf_elems > 0) {
    // One copy out per buffer, after which it goes back to the allocator.
    const size_t nb = static_cast<size_t>(pf_elems) * sizeof(float);
    mark_first_out();
    CTD_CHECK(ember_memcpy_async(hm, pf_m, nb, 1, ds));
    CTD_CHECK(ember_memcpy_async(hv, pf_v, nb, 1, ds));
    CTD_CHECK(ember_event_record(ev_pf_drained_, ds));
    runtime::release_after(ev_pf_drained_, {pf_m_.storage(), pf_v_.storage()});
    pf_m_ = Tensor{};
    pf_v_ = Tensor{};
    pf_elems_ = 0;
    bytes_out += 2.0 * static_cast<double>(nb);
  }
  if (first_out) CTD_CHECK(ember_event_record(ev_d2h_begin_, ds));  // nothing was moved
  CTD_CHECK(ember_event_record(ev_done_, ds));
  // Only now, after the last data_ptr() above: later users of a parameter or
  // its gradient on the compute stream wait for that parameter's update.
  for (size_t j = 0; j < layout_.size(); ++j) {
    if (!work[j].p) continue;
    Tensor& p = groups_[layout_[j].gi].params[layout_[j].pi];
    p.storage()->set_ready_event(ev_param_[layout_[j].gi][layout_[j].pi]);
    p.grad().storage()->set_ready_event(ev_param_[layout_[j].gi][layout_[j].pi]);
  }
  in_flight_ = true;
  stats_.last_h2d_bytes = bytes_in;
  stats_.last_d2h_bytes = bytes_out;
  stats_.last_prefetch_bytes = bytes_out - bytes_in;
  stats_.last_skipped_bytes = skipped;
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
    std::vector<float*> wptrs;
    wptrs.reserve(grads.size());
    for (auto& g : grads) wptrs.push_back(fp(g));
    const size_t swb = ember_scale_multi_workspace_bytes(count);
    Tensor sws = swb ? workspace(swb) : Tensor{};
    CTD_CHECK(ember_scale_multi(wptrs.data(), sizes.data(), count, scale,
                                swb ? sws.data_ptr() : nullptr, swb, S()));
  }
  return total;
}

}  // namespace ctd::optim
