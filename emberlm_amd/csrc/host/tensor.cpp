// Tensor construction, host transfers and views.
// Reference: src/core/tensor.cpp:17-130.  Host<->device copies are enqueued on
// the compute stream and waited for, so they are ordered after every kernel
// that produced the data (the reference relied on the legacy default stream).
#include <cstring>
#include <stdexcept>
#include <string>

#include "ctd/autograd.h"
#include "ctd/runtime.h"
#include "ctd/tensor.h"

namespace ctd {

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape) {
  std::vector<int64_t> s(shape.size(), 1);
  for (int64_t i = static_cast<int64_t>(shape.size()) - 2; i >= 0; --i) s[i] = s[i + 1] * shape[i + 1];
  return s;
}

namespace {

// Gradient of a reshape view: the same values in the input's shape.
class ReshapeBackward : public autograd::Node {
 public:
  std::vector<int64_t> input_shape;
  std::vector<Tensor> backward(const std::vector<Tensor>& grads_out) override {
    return {grads_out.at(0).reshape(input_shape)};
  }
  const char* name() const override { return "ReshapeBackward"; }
};

[[noreturn]] void placeholder_access() {
  throw std::runtime_error(
      "tensor values are not computed: this tensor only carries autograd history "
      "(a recompute placeholder); use it for backward() only");
}

int64_t shape_numel(const std::vector<int64_t>& shape) {
  int64_t n = 1;
  for (auto d : shape) {
    if (d < 0) throw std::runtime_error("Tensor: negative dimension");
    n *= d;
  }
  return n;
}
}  // namespace

Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype, Device device) {
  Tensor t;
  const size_t nbytes = static_cast<size_t>(shape_numel(shape)) * dtype_size(dtype);
  t.storage_ = make_storage(nbytes, allocator_for(device));
  t.strides_ = contiguous_strides(shape);
  t.shape_ = std::move(shape);
  t.dtype_ = dtype;
  t.device_ = device;
  return t;
}

Tensor Tensor::zeros(std::vector<int64_t> shape, DType dtype, Device device) {
  Tensor t = empty(std::move(shape), dtype, device);
  const size_t nb = t.nbytes();
  if (nb == 0) return t;
  if (device.is_hip()) {
    if (nb % 4 == 0) {
      CTD_CHECK(ember_fill(static_cast<float*>(t.data_ptr()), static_cast<int64_t>(nb / 4), 0.0f,
                           runtime::compute_stream()));
    } else {
      std::vector<unsigned char> z(nb, 0);
      CTD_CHECK(ember_memcpy_async(t.data_ptr(), z.data(), nb, 0, runtime::compute_stream()));
      runtime::synchronize();
    }
  } else {
    std::memset(t.data_ptr(), 0, nb);
  }
  return t;
}

Tensor Tensor::zeros_pinned(std::vector<int64_t> shape, DType dtype) {
  Tensor t;
  const size_t nbytes = static_cast<size_t>(shape_numel(shape)) * dtype_size(dtype);
  t.storage_ = make_storage(nbytes, pinned_cpu_allocator());
  if (nbytes) std::memset(t.storage_->data(), 0, nbytes);
  t.strides_ = contiguous_strides(shape);
  t.shape_ = std::move(shape);
  t.dtype_ = dtype;
  t.device_ = kCPU;
  return t;
}

Tensor Tensor::from_host(const void* host_data, std::vector<int64_t> shape, DType dtype,
                         Device device) {
  Tensor t = empty(std::move(shape), dtype, device);
  const size_t nb = t.nbytes();
  if (nb == 0) return t;
  if (!host_data) throw std::runtime_error("from_host: null host pointer");
  if (device.is_hip()) {
    CTD_CHECK(ember_memcpy_async(t.data_ptr(), host_data, nb, 0, runtime::compute_stream()));
    runtime::synchronize();
  } else {
    std::memcpy(t.data_ptr(), host_data, nb);
  }
  return t;
}

void Tensor::copy_to_host(void* dst) const {
  if (placeholder_) placeholder_access();
  if (!is_contiguous()) throw std::runtime_error("copy_to_host: tensor must be contiguous");
  const size_t nb = nbytes();
  if (nb == 0) return;
  if (device_.is_hip()) {
    CTD_CHECK(ember_memcpy_async(dst, data_ptr(), nb, 1, runtime::compute_stream()));
    runtime::synchronize();
  } else {
    std::memcpy(dst, data_ptr(), nb);
  }
}

Tensor Tensor::reshape(std::vector<int64_t> new_shape) const {
  if (!is_contiguous()) throw std::runtime_error("reshape: tensor must be contiguous");
  int64_t infer = -1, known = 1;
  for (size_t i = 0; i < new_shape.size(); ++i) {
    if (new_shape[i] == -1) {
      if (infer >= 0) throw std::runtime_error("reshape: more than one -1");
      infer = static_cast<int64_t>(i);
    } else {
      known *= new_shape[i];
    }
  }
  if (infer >= 0) new_shape[infer] = known ? numel() / known : 0;
  if (shape_numel(new_shape) != numel()) {
    std::string m = "reshape: numel mismatch (" + std::to_string(numel()) + " vs " +
                    std::to_string(shape_numel(new_shape)) + ")";
    throw std::runtime_error(m);
  }
  Tensor t;
  t.storage_ = storage_;
  t.storage_offset_ = storage_offset_;
  t.strides_ = contiguous_strides(new_shape);
  t.shape_ = std::move(new_shape);
  t.dtype_ = dtype_;
  t.device_ = device_;
  t.placeholder_ = placeholder_;
  // ReshapeBackward as in src/core/tensor.cpp:17-25, 124-129 of the reference.
  if (autograd::any_requires_grad({*this})) {
    auto node = std::make_shared<ReshapeBackward>();
    node->input_shape = shape_;
    node->next_edges = autograd::collect_next_edges({*this});
    autograd::set_history(t, std::move(node));
  }
  return t;
}

Tensor Tensor::view_at(int64_t offset, std::vector<int64_t> shape) const {
  if (!is_contiguous()) throw std::runtime_error("view_at: tensor must be contiguous");
  if (offset < 0 || offset + shape_numel(shape) > numel())
    throw std::runtime_error("view_at: view out of range");
  Tensor t;
  t.storage_ = storage_;
  t.storage_offset_ = storage_offset_ + offset;
  t.strides_ = contiguous_strides(shape);
  t.shape_ = std::move(shape);
  t.dtype_ = dtype_;
  t.device_ = device_;
  t.placeholder_ = placeholder_;
  return t;
}

int64_t Tensor::numel() const { return shape_numel(shape_); }

bool Tensor::is_contiguous() const { return strides_ == contiguous_strides(shape_); }

void* Tensor::data_ptr() {
  if (placeholder_) placeholder_access();
  if (!storage_) return nullptr;
  if (storage_->ready_event()) runtime::wait_ready(*storage_);
  return static_cast<char*>(storage_->data()) + storage_offset_ * dtype_size(dtype_);
}

const void* Tensor::data_ptr() const {
  if (placeholder_) placeholder_access();
  if (!storage_) return nullptr;
  if (storage_->ready_event()) runtime::wait_ready(*storage_);
  return static_cast<const char*>(storage_->data()) + storage_offset_ * dtype_size(dtype_);
}

}  // namespace ctd
