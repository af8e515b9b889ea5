#pragma once
// Placement policy of the caching device allocator, independent of where the
// memory comes from: segments are obtained from a backend (hipMalloc on the
// GPU, a counter when a recorded allocation history is replayed on the host),
// cut into blocks, and freed blocks are merged with free address neighbours.
//
// The reference allocates every tensor with cudaMalloc and frees it with
// cudaFree (src/core/allocator.cpp:14-30): its footprint is its live tensors,
// at the price of a driver call (and an implicit device synchronisation on
// free) per tensor.  This arena keeps freed memory for reuse without the
// driver, so what it holds must stay close to what is live: a request is
// served from the smallest free block that fits (lowest address among equal
// sizes), the rest of that block stays free, and a freed block coalesces with
// free neighbours of the same segment, so memory freed by one tensor shape
// serves any other.  Requests up to kSmallRequest come from their own small
// segments, so that long-lived small tensors (norm weights, scalars) do not
// pin large segments.

#include <cstddef>
#include <cstdint>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

namespace ctd::detail {

class ArenaBackend {
 public:
  virtual ~ArenaBackend() = default;
  // Obtains `bytes` of device memory at *base (false: out of memory).
  virtual bool obtain(size_t bytes, uintptr_t* base) = 0;
  // Returns a segment obtained earlier.  Called only after quiesce().
  virtual void give_back(uintptr_t base, size_t bytes) = 0;
  // Waits until no queued device work can still touch freed blocks.
  virtual void quiesce() = 0;
};

struct ArenaStats {
  size_t live_bytes = 0;        // bytes in blocks handed out
  size_t peak_live_bytes = 0;
  size_t held_bytes = 0;        // bytes in segments (live + cached)
  size_t peak_held_bytes = 0;
  int64_t segments_obtained = 0;
  int64_t trims = 0;            // times the cache was emptied to satisfy a request
  int64_t segments = 0;         // segments held now
};

class BlockArena {
 public:
  static constexpr size_t kGranule = 512;                  // block size multiple
  static constexpr size_t kSmallRequest = size_t{1} << 20;  // small pool up to this
  static constexpr size_t kSmallSegment = size_t{2} << 20;
  static constexpr size_t kLargeSegmentGranule = size_t{2} << 20;

  explicit BlockArena(ArenaBackend& backend) : backend_(backend) {}
  ~BlockArena();
  BlockArena(const BlockArena&) = delete;
  BlockArena& operator=(const BlockArena&) = delete;

  // Hands out at least `bytes` (> 0) bytes, 512-byte aligned.  Throws
  // std::runtime_error when neither the cache nor the backend can serve it,
  // or when serving it would take the held bytes past the limit even after
  // the cache has been emptied.
  uintptr_t allocate(size_t bytes);
  // Returns the block at `addr` (from allocate) to the cache; returns its
  // size, or 0 for an address this arena did not hand out.
  size_t release(uintptr_t addr);
  // Quiesces the device and gives every segment without a live block back.
  void trim();

  // Upper bound on held bytes (0: none).  Exceeding it first empties the
  // cache (counted in ArenaStats::trims), then fails the request.
  void set_limit(size_t bytes) { limit_ = bytes; }
  size_t limit() const { return limit_; }

  const ArenaStats& stats() const { return stats_; }
  void reset_peaks() {
    stats_.peak_live_bytes = stats_.live_bytes;
    stats_.peak_held_bytes = stats_.held_bytes;
  }
  // Size of the largest free block (0 if none).
  size_t largest_free() const;
  // Whether a cached free block serves a request of `bytes` (no new segment).
  bool fits(size_t bytes) const;
  // `want` when a free block holds it or none holds `least`; else the
  // largest free block (a multiple of kGranule).  See elastic_workspace_bytes.
  size_t elastic_fit(size_t want, size_t least) const {
    const size_t largest = largest_free() / kGranule * kGranule;
    return largest >= want || largest < least ? want : largest;
  }
  // Pieces (byte sizes, each a whole number of `unit`s) for a workspace
  // that may be split: the largest free blocks are taken first, each for as
  // many units as it holds, until `want` units are placed or `max_pieces`
  // blocks are used, then cut to a multiple of `multiple` units when that
  // leaves at least one multiple.  Fewer than `least` units placed that way:
  // one more piece for the rest of `least`, which grows the arena.  See
  // device_scatter_plan.
  std::vector<size_t> scatter_fit(size_t unit, size_t want, size_t least, size_t multiple,
                                  size_t max_pieces) const;
  // (address, size) of every block handed out, in address order.
  std::vector<std::pair<uintptr_t, size_t>> live_blocks() const;

 private:
  struct Segment;
  struct Block {
    uintptr_t addr;
    size_t size;
    Segment* seg;
    Block* lo;   // address neighbours inside the segment
    Block* hi;
    bool free;
  };
  struct Segment {
    uintptr_t base;
    size_t size;
    bool small;
    size_t live = 0;  // blocks handed out
  };
  struct BySize {
    bool operator()(const Block* a, const Block* b) const {
      return a->size != b->size ? a->size < b->size : a->addr < b->addr;
    }
  };
  using FreeSet = std::set<Block*, BySize>;

  static size_t round_request(size_t bytes) {
    return (bytes + kGranule - 1) / kGranule * kGranule;
  }
  FreeSet& pool(bool small) { return small ? free_small_ : free_large_; }
  Block* take_fit(FreeSet& set, size_t size);
  Block* grow(bool small, size_t size);
  Block* carve(Block* b, size_t size);
  void give_back_free_segments();

  ArenaBackend& backend_;
  FreeSet free_small_, free_large_;
  std::unordered_map<uintptr_t, Block*> live_;
  std::vector<Segment*> segments_;
  ArenaStats stats_;
  size_t limit_ = 0;
};

// Replays an allocation history recorded by the device allocator (lines
// "a <id> <bytes>", "f <id>", "m <label>", and "e <want> <least>" before a
// workspace whose size followed elastic_fit: the replay asks its own arena
// and allocates that answer instead of the recorded size; "s <unit> <want>
// <least> <multiple> <max_pieces> <count>" before the `count` pieces of a split
// workspace planned by scatter_fit: the replay plans and allocates its own
// pieces and frees them with the first recorded one) on a BlockArena
// whose backend only counts addresses, so a placement policy can be judged
// on a real training step's requests without a GPU.  Returns the arena's
// statistics at the end.
ArenaStats replay_history(const std::string& path, size_t limit);

}  // namespace ctd::detail
