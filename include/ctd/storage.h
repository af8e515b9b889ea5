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

  // An event (ember_event_t) recorded on another stream after work that
  // writes this buffer, e.g. the offloaded optimizer's update of a parameter.
  // Tensor::data_ptr() makes the compute stream wait for it on first access
  // and clears it, so the buffer's next user is ordered after that writer.
  void set_ready_event(void* ev) { ready_event_ = ev; }
  void* ready_event() const { return ready_event_; }
  void* take_ready_event() {
    void* e = ready_event_;
    ready_event_ = nullptr;
    return e;
  }

 private:
  void release_() noexcept;

  Allocator* allocator_ = nullptr;
  void* data_ = nullptr;
  size_t nbytes_ = 0;
  Device device_{};
  bool pinned_ = false;
  void* ready_event_ = nullptr;
};

using StoragePtr = std::shared_ptr<Storage>;

inline StoragePtr make_storage(size_t nbytes, Allocator& alloc) {
  return std::make_shared<Storage>(nbytes, alloc);
}

}  // namespace ctd
