#pragma once
// Raw byte buffer on a device (mirrors include/ctd/storage.h of the reference).

#include <cstddef>
#include <memory>

#include "ctd/allocator.h"
#include "ctd/device.h"

namespace ctd {

class Storage {
 public:
  Storage(size_t nbytes, Allocator& allocator);

  Storage(const Storage&) = delete;
  Storage& operator=(const Storage&) = delete;
  Storage(Storage&& other) noexcept;
  Storage& operator=(Storage&& other) noexcept;
  ~Storage();

  void* data() { return data_; }
  const void* data() const { return data_; }
  size_t nbytes() const { return nbytes_; }
  const Device& device() const { return device_; }
  bool pinned() const { return pinned_; }

 private:
  void release_() noexcept;

  Allocator* allocator_ = nullptr;
  void* data_ = nullptr;
  size_t nbytes_ = 0;
  Device device_{};
  bool pinned_ = false;
};

using StoragePtr = std::shared_ptr<Storage>;

inline StoragePtr make_storage(size_t nbytes, Allocator& alloc) {
  return std::make_shared<Storage>(nbytes, alloc);
}

}  // namespace ctd
