#pragma once
// Memory allocators (interface of include/ctd/allocator.h in the reference).
//
// hip_allocator() is a caching device allocator: memory obtained from hipMalloc
// in segments is cut into blocks, a request takes the smallest free block that
// fits (the rest stays free), and freed blocks merge with free neighbours, so
// the training loop reaches neither hipMalloc nor hipFree (which would
// synchronise the device) once its working set is in place.  All device work
// is ordered on one compute stream, so a block freed on the host can be
// handed out again at once.

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

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
  size_t reserved_bytes = 0;        // bytes held from the driver: allocated + cached
  size_t peak_reserved_bytes = 0;
  int64_t num_device_mallocs = 0;   // segments obtained from the driver
  int64_t num_cache_flushes = 0;    // times cached segments went back to satisfy a request
  // hipMemGetInfo's total - free: everything the device holds for the process
  // (reserved bytes, buffers outside the allocator, the runtime's own), as
  // last sampled and its highest sample since reset_peak_device_memory().
  // Sampled whenever the allocator obtains a segment and by
  // sample_device_memory().
  size_t device_used_bytes = 0;
  size_t peak_device_used_bytes = 0;
  size_t limit_bytes = 0;           // set_device_memory_limit (0: none)
  size_t largest_free_block = 0;
};

DeviceMemoryStats device_memory_stats();
void reset_peak_device_memory();
// Returns cached free segments to the driver (synchronises the device).
void empty_device_cache();
// Caps the bytes the allocator holds from the driver (0: no cap).  A request
// that cannot be served within it empties the cache (counted in
// num_cache_flushes) and, if that does not make room, throws.
void set_device_memory_limit(size_t bytes);
// Takes a hipMemGetInfo sample into device_used_bytes / its peak.
void sample_device_memory();
// Size for a scratch buffer that works with anything from `least` to `want`
// bytes (a chunked computation whose chunk count follows the buffer): `want`
// when a cached free block can hold it (or when none holds `least` either, so
// the allocator would grow anyway), else the largest cached free block.  Lets
// large workspaces fill the holes that other tensors' lifetimes leave instead
// of growing the device memory held.
size_t elastic_workspace_bytes(size_t want, size_t least);
// Byte sizes of the pieces for a workspace that may be split into separate
// allocations of whole `unit`s (the rows of a chunked computation): up to
// `want` units from the largest cached free blocks, at most `max_pieces`
// pieces, cut to a multiple of `multiple` units when short of `want`; when
// those hold fewer than `least` units, one more piece for the rest of
// `least`, which grows the memory held.  Allocate the pieces in the order
// given, before any other allocation, for them to land where planned.
std::vector<size_t> device_scatter_plan(size_t unit, size_t want, size_t least, size_t multiple,
                                        size_t max_pieces);
// Allocation history for offline study of the allocator's placement: start
// records the blocks live now and then every request and release; stop
// writes the record to `path` (lines "a <id> <bytes>", "f <id>", "m <label>").
void start_allocation_history();
void mark_allocation_history(const std::string& label);
void stop_allocation_history(const std::string& path);
// Pinned host bytes currently allocated.
size_t pinned_host_bytes();

}  // namespace ctd
