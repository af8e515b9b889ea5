#pragma once
// Tensor (mirrors include/ctd/tensor.h of the reference): a (storage, layout,
// dtype) triple with strides in elements; views share one Storage.

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

#include "ctd/device.h"
#include "ctd/dtype.h"
#include "ctd/storage.h"

namespace ctd {

namespace autograd { struct AutogradMeta; }

class Tensor {
 public:
  Tensor() = default;

  static Tensor empty(std::vector<int64_t> shape, DType dtype, Device device);
  static Tensor zeros(std::vector<int64_t> shape, DType dtype, Device device);
  // Page-locked host memory (hipHostMalloc).
  static Tensor zeros_pinned(std::vector<int64_t> shape, DType dtype);
  static Tensor from_host(const void* host_data, std::vector<int64_t> shape, DType dtype,
                          Device device);

  // Synchronous copy of the whole tensor to host memory.
  void copy_to_host(void* dst) const;

  // Zero-copy view with a new shape. Tensor must be contiguous.
  Tensor reshape(std::vector<int64_t> new_shape) const;
  // Contiguous view of prod(shape) elements starting `offset` elements into
  // this contiguous tensor; shares the storage, carries no autograd history.
  Tensor view_at(int64_t offset, std::vector<int64_t> shape) const;

  const std::vector<int64_t>& shape() const { return shape_; }
  const std::vector<int64_t>& strides() const { return strides_; }
  int64_t dim() const { return static_cast<int64_t>(shape_.size()); }
  int64_t numel() const;
  size_t nbytes() const { return static_cast<size_t>(numel()) * dtype_size(dtype_); }

  DType dtype() const { return dtype_; }
  const Device& device() const { return device_; }
  bool is_contiguous() const;
  bool defined() const { return storage_ != nullptr; }

  void* data_ptr();
  const void* data_ptr() const;

  const StoragePtr& storage() const { return storage_; }
  int64_t storage_offset() const { return storage_offset_; }

  // A tensor that carries autograd history but whose elements are not its
  // values (the recompute form of a checkpointed block's output, the product
  // node of a GEMM fused with an add): backward() works through it, while
  // data_ptr() and copy_to_host() throw.  Views of it are placeholders too.
  // Added in this build.
  bool is_placeholder() const { return placeholder_; }
  Tensor& mark_placeholder() {
    placeholder_ = true;
    return *this;
  }

  // Autograd interface.
  Tensor& requires_grad_(bool v = true);
  bool requires_grad() const;
  Tensor grad() const;
  void zero_grad_();
  void backward();
  void backward(const Tensor& grad_output);
  // retain_graph = true keeps the graph (nodes and their saved tensors) so
  // that another backward can run through it, as the reference's engine
  // always does (src/core/autograd.cu:158-237); the default releases each
  // node as soon as it has run.
  void backward(bool retain_graph);
  void backward(const Tensor& grad_output, bool retain_graph);
  Tensor detach() const;

  const std::shared_ptr<autograd::AutogradMeta>& autograd_meta() const { return autograd_meta_; }
  std::shared_ptr<autograd::AutogradMeta>& mutable_autograd_meta() { return autograd_meta_; }

 private:
  StoragePtr storage_;
  std::vector<int64_t> shape_;
  std::vector<int64_t> strides_;
  int64_t storage_offset_ = 0;
  DType dtype_ = DType::kFloat32;
  Device device_{};
  std::shared_ptr<autograd::AutogradMeta> autograd_meta_;
  bool placeholder_ = false;
};

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape);

}  // namespace ctd
