#pragma once
// Memory allocators (interface of include/ctd/allocator.h in the reference).
//
// hip_allocator() is a caching device allocator: freed blocks are kept in
// per-size free lists and reused (no hipFree, and therefore no implicit device
// synchronisation, in the training loop), and it records the high-water mark of
// live bytes.  All device work is ordered on one compute stream, so a block
// freed on the host can be handed out again at once.

#include <cstddef>
#include <cstdint>

#include "ctd/device.h"

namespace ctd {

class Allocator {
 public:
  virtual ~Allocator() = default;
  virtual void* allocate(size_t nbytes) = 0;
  virtual void deallocate(void* ptr) noexcept = 0;
  virtual Device device() const = 0;
};

Allocator& hip_allocator();
Allocator& cpu_allocator();
Allocator& pinned_cpu_allocator();
Allocator& allocator_for(const Device& device);

struct DeviceMemoryStats {
  size_t allocated_bytes = 0;       // live bytes handed out
  size_t peak_allocated_bytes = 0;  // high-water mark of allocated_bytes
  size_t reserved_bytes = 0;        // allocated + cached in free lists
  size_t peak_reserved_bytes = 0;
  int64_t num_device_mallocs = 0;   // calls that reached the driver
};

DeviceMemoryStats device_memory_stats();
void reset_peak_device_memory();
// Returns cached free blocks to the driver.
void empty_device_cache();
// Pinned host bytes currently allocated.
size_t pinned_host_bytes();

}  // namespace ctd
