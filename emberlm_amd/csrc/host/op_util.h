// Helpers shared by the op implementations (host side, private).
#pragma once

#include <stdexcept>
#include <string>

#include "ctd/autograd.h"
#include "ctd/runtime.h"
#include "ctd/tensor.h"

namespace ctd::ops::detail {

inline ember_stream_t S() { return runtime::compute_stream(); }

inline void require(bool cond, const std::string& msg) {
  if (!cond) throw std::runtime_error(msg);
}

// fp32, on the GPU, contiguous: the preconditions every kernel wrapper checks
// before launch (the reference's *_impl checks, e.g. src/ops/norm.cu:110-120).
inline void check_f32(const Tensor& t, const char* op, const char* what = "input") {
  require(t.defined(), std::string(op) + ": " + what + " is undefined");
  require(t.dtype() == DType::kFloat32, std::string(op) + ": " + what + " must be float32");
  require(t.device().is_hip(), std::string(op) + ": " + what + " must be on the HIP device");
  require(t.is_contiguous(), std::string(op) + ": " + what + " must be contiguous");
}

inline float* fp(Tensor& t) { return static_cast<float*>(t.data_ptr()); }
inline const float* cfp(const Tensor& t) { return static_cast<const float*>(t.data_ptr()); }

inline Tensor empty_like(const Tensor& t) { return Tensor::empty(t.shape(), t.dtype(), t.device()); }

// Drops a backward node's saved tensors once it has run, unless the backward
// pass retains its graph for another pass (autograd::graph_retained()).
template <typename... Ts>
void release_saved(Ts&... ts) {
  if (!autograd::graph_retained()) ((ts = Tensor{}), ...);
}

// Scratch buffer from the caching allocator (freed when the returned tensor dies).
inline Tensor workspace(size_t bytes) {
  return Tensor::empty({static_cast<int64_t>((bytes + 3) / 4)}, DType::kFloat32, kHIP0);
}

}  // namespace ctd::ops::detail
