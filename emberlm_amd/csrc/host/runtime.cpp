// Runtime glue, allocators and Storage.
//
// Reference: src/core/allocator.cpp:14-57 (raw cudaMalloc/cudaFree per tensor,
// malloc CPU allocator, cudaMallocHost pinned allocator) and
// src/core/storage.cpp.  The device allocator here keeps freed memory for
// reuse (BlockArena: best fit, split, coalesce) so the training loop never
// reaches the driver after its first step (hipFree would also synchronise the
// device), and it records the high-water marks of live bytes, of bytes held
// from the driver, and of the device's used memory (hipMemGetInfo, sampled
// whenever a segment is obtained and at the callers' phase boundaries).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "ctd/allocator.h"
#include "ctd/runtime.h"
#include "ctd/storage.h"
#include "block_arena.h"

namespace ctd {

namespace runtime {

void check(int status, const char* what) {
  if (status != EMBER_OK)
    throw std::runtime_error(std::string(what) + ": " + ember_status_string(status));
}

namespace {
struct Streams {
  ember_stream_t compute = nullptr, h2d = nullptr, d2h = nullptr;
  Streams() {
    check(ember_stream_create(&compute), "create compute stream");
    check(ember_stream_create(&h2d), "create h2d stream");
    check(ember_stream_create(&d2h), "create d2h stream");
  }
};
Streams& streams() {
  static Streams s;
  return s;
}
}  // namespace

ember_stream_t compute_stream() { return streams().compute; }
ember_stream_t h2d_stream() { return streams().h2d; }
ember_stream_t d2h_stream() { return streams().d2h; }

void synchronize() { check(ember_stream_synchronize(compute_stream()), "synchronize"); }

void wait_ready(Storage& s) {
  if (void* e = s.take_ready_event()) check(ember_stream_wait_event(compute_stream(), e), "wait_ready");
}

namespace {
struct Deferred {
  std::mutex mu;
  std::vector<std::pair<ember_event_t, std::vector<StoragePtr>>> items;
};
Deferred& deferred() {
  static Deferred d;
  return d;
}
}  // namespace

void release_after(ember_event_t done, std::vector<StoragePtr> keep) {
  Deferred& d = deferred();
  std::lock_guard<std::mutex> lk(d.mu);
  d.items.emplace_back(done, std::move(keep));
}

size_t collect_released() {
  Deferred& d = deferred();
  std::vector<std::vector<StoragePtr>> drop;
  size_t left = 0;
  {
    std::lock_guard<std::mutex> lk(d.mu);
    if (d.items.empty()) return 0;
    auto it = d.items.begin();
    while (it != d.items.end()) {
      const int rc = ember_event_query(it->first);
      if (rc == EMBER_OK) {
        drop.push_back(std::move(it->second));
        it = d.items.erase(it);
      } else {
        if (rc != EMBER_NOTREADY) check(rc, "release_after event");
        ++it;
      }
    }
    left = d.items.size();
  }
  return left;  // `drop` releases its storages here, outside the lock
}

void drain_released() {
  Deferred& d = deferred();
  std::vector<std::pair<ember_event_t, std::vector<StoragePtr>>> items;
  {
    std::lock_guard<std::mutex> lk(d.mu);
    items.swap(d.items);
  }
  for (auto& [e, keep] : items) {
    check(ember_event_synchronize(e), "drain_released");
    keep.clear();
  }
}

bool wait_oldest_released() {
  Deferred& d = deferred();
  std::pair<ember_event_t, std::vector<StoragePtr>> item;
  {
    std::lock_guard<std::mutex> lk(d.mu);
    if (d.items.empty()) return false;
    item = std::move(d.items.front());
    d.items.erase(d.items.begin());
  }
  check(ember_event_synchronize(item.first), "wait_oldest_released");
  item.second.clear();
  return true;
}

bool device_available() {
  int n = 0;
  return ember_get_device_count(&n) == EMBER_OK && n > 0;
}

namespace {
struct GemmProfiler {
  std::mutex mu;
  bool on = false;
  std::vector<ember_event_t> pool;                       // free events
  std::vector<std::pair<ember_event_t, ember_event_t>> spans;
  std::vector<double> flops;
  std::vector<int> variant;
  // Launches sized on the device: flops = per_row * clamp(slot - base, 0, max)
  // with the row count copied into a device slot when the launch is queued.
  struct DynRows {
    size_t span;
    int64_t slot, base, max;
    double per_row;
  };
  std::vector<DynRows> dyn;
  int64_t* slots = nullptr;  // kSlots int64 on the device, allocated on first use
  static constexpr int64_t kSlots = 1 << 16;
  ember_event_t get() {
    if (!pool.empty()) {
      ember_event_t e = pool.back();
      pool.pop_back();
      return e;
    }
    ember_event_t e = nullptr;
    check(ember_event_create(&e), "gemm profiler event");
    return e;
  }
};
GemmProfiler& prof() {
  static GemmProfiler* p = new GemmProfiler();
  return *p;
}
}  // namespace

void gemm_profile_enable(bool on) {
  std::lock_guard<std::mutex> lk(prof().mu);
  prof().on = on;
}
bool gemm_profiling() { return prof().on; }

void* gemm_profile_begin() {
  auto& p = prof();
  if (!p.on) return nullptr;
  std::lock_guard<std::mutex> lk(p.mu);
  ember_event_t e = p.get();
  check(ember_event_record(e, compute_stream()), "gemm profiler record");
  return e;
}

void gemm_profile_end(void* begin, double flops, int variant) {
  if (!begin) return;
  auto& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  ember_event_t e = p.get();
  check(ember_event_record(e, compute_stream()), "gemm profiler record");
  p.spans.emplace_back(begin, e);
  p.flops.push_back(flops);
  p.variant.push_back(variant >= 0 && variant < kProfileVariants ? variant : 0);
}

void gemm_profile_end_rows(void* begin, double flops_per_row, const int64_t* count,
                           int64_t base, int64_t max_rows, int variant) {
  if (!begin) return;
  auto& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  if (!p.slots)
    check(ember_device_malloc(reinterpret_cast<void**>(&p.slots),
                              GemmProfiler::kSlots * sizeof(int64_t)),
          "gemm profiler slots");
  if (static_cast<int64_t>(p.dyn.size()) >= GemmProfiler::kSlots)
    throw std::runtime_error("gemm profiler: too many device-sized launches between collects");
  const int64_t slot = static_cast<int64_t>(p.dyn.size());
  check(ember_memcpy_async(p.slots + slot, count, sizeof(int64_t), 2, compute_stream()),
        "gemm profiler count copy");
  ember_event_t e = p.get();
  check(ember_event_record(e, compute_stream()), "gemm profiler record");
  p.dyn.push_back({p.spans.size(), slot, base, max_rows, flops_per_row});
  p.spans.emplace_back(begin, e);
  p.flops.push_back(0.0);
  p.variant.push_back(variant >= 0 && variant < kProfileVariants ? variant : 0);
}

void gemm_profile_collect(int64_t* launches, double* flops, double* total_ms) {
  auto& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  synchronize();
  if (!p.dyn.empty()) {
    std::vector<int64_t> counts(p.dyn.size());
    check(ember_memcpy(counts.data(), p.slots, counts.size() * sizeof(int64_t), 1),
          "gemm profiler counts");
    for (const auto& d : p.dyn) {
      const int64_t rows = std::min(std::max<int64_t>(counts[d.slot] - d.base, 0), d.max);
      p.flops[d.span] = d.per_row * static_cast<double>(rows);
    }
    p.dyn.clear();
  }
  for (int v = 0; v < kProfileVariants; ++v) {
    launches[v] = 0;
    flops[v] = 0.0;
    total_ms[v] = 0.0;
  }
  for (size_t i = 0; i < p.spans.size(); ++i) {
    float t = 0.f;
    check(ember_event_elapsed_ms(&t, p.spans[i].first, p.spans[i].second), "gemm profiler elapsed");
    const int v = p.variant[i];
    launches[v] += 1;
    flops[v] += p.flops[i];
    total_ms[v] += t;
    p.pool.push_back(p.spans[i].first);
    p.pool.push_back(p.spans[i].second);
  }
  p.spans.clear();
  p.flops.clear();
  p.variant.clear();
}

}  // namespace runtime

namespace {

// Device memory through BlockArena (best fit, split, coalesce) over hipMalloc.
class HipBackend final : public detail::ArenaBackend {
 public:
  bool obtain(size_t bytes, uintptr_t* base) override {
    void* p = nullptr;
    if (ember_device_malloc(&p, bytes) != EMBER_OK) return false;
    *base = reinterpret_cast<uintptr_t>(p);
    return true;
  }
  void give_back(uintptr_t base, size_t) override {
    ember_device_free(reinterpret_cast<void*>(base));
  }
  // Blocks are freed on the host while kernels queued earlier may still read
  // them; a segment goes back to the driver only once the device is idle.
  void quiesce() override { ember_device_synchronize(); }
};

class HipCachingAllocator final : public Allocator {
 public:
  HipCachingAllocator() : arena_(backend_) {}

  void* allocate(size_t nbytes) override {
    if (nbytes == 0) return nullptr;
    // Blocks a side stream has finished with go back first.  If some are
    // still in use and this request would set a new lifetime high-water mark
    // of live bytes, or needs a new large segment (no cached block holds it), wait
    // for them, oldest first, until it fits: the host runs ahead of the GPU,
    // and the side stream's buffers (gradients the offloaded update still
    // reads, released in the order the update reaches them) would otherwise
    // count on top of the next forward's own peak or make the arena grow.
    while (runtime::collect_released() > 0) {
      bool wait;
      {
        std::lock_guard<std::mutex> lk(mu_);
        wait = arena_.stats().live_bytes + nbytes > high_water_ ||
               (nbytes > detail::BlockArena::kSmallRequest && !arena_.fits(nbytes));
      }
      if (!wait || !runtime::wait_oldest_released()) break;
    }
    std::lock_guard<std::mutex> lk(mu_);
    const int64_t segments_before = arena_.stats().segments_obtained;
    const uintptr_t a = arena_.allocate(nbytes);
    const detail::ArenaStats& st = arena_.stats();
    high_water_ = std::max(high_water_, st.live_bytes);
    if (st.segments_obtained != segments_before) sample_locked();
    if (tracing_) {
      const uint64_t id = next_id_++;
      trace_ids_[a] = id;
      trace_ << "a " << id << ' ' << nbytes << '\n';
    }
    return reinterpret_cast<void*>(a);
  }

  void deallocate(void* ptr) noexcept override {
    if (!ptr) return;
    std::lock_guard<std::mutex> lk(mu_);
    const uintptr_t a = reinterpret_cast<uintptr_t>(ptr);
    if (arena_.release(a) == 0) return;
    if (tracing_) {
      auto it = trace_ids_.find(a);
      if (it != trace_ids_.end()) {
        trace_ << "f " << it->second << '\n';
        trace_ids_.erase(it);
      }
    }
  }

  Device device() const override { return kHIP0; }

  DeviceMemoryStats stats() {
    std::lock_guard<std::mutex> lk(mu_);
    const detail::ArenaStats& a = arena_.stats();
    DeviceMemoryStats s;
    s.allocated_bytes = a.live_bytes;
    s.peak_allocated_bytes = a.peak_live_bytes;
    s.reserved_bytes = a.held_bytes;
    s.peak_reserved_bytes = a.peak_held_bytes;
    s.num_device_mallocs = a.segments_obtained;
    s.num_cache_flushes = a.trims;
    s.device_used_bytes = device_used_;
    s.peak_device_used_bytes = peak_device_used_;
    s.limit_bytes = arena_.limit();
    s.largest_free_block = arena_.largest_free();
    return s;
  }
  void reset_peak() {
    std::lock_guard<std::mutex> lk(mu_);
    arena_.reset_peaks();
    peak_device_used_ = 0;
    sample_locked();
  }
  void empty_cache() {
    std::lock_guard<std::mutex> lk(mu_);
    arena_.trim();
  }
  void set_limit(size_t bytes) {
    std::lock_guard<std::mutex> lk(mu_);
    arena_.set_limit(bytes);
  }
  void sample() {
    std::lock_guard<std::mutex> lk(mu_);
    sample_locked();
  }
  std::vector<size_t> scatter_plan(size_t unit, size_t want, size_t least, size_t multiple,
                                   size_t max_pieces) {
    std::lock_guard<std::mutex> lk(mu_);
    std::vector<size_t> pieces = arena_.scatter_fit(unit, want, least, multiple, max_pieces);
    if (tracing_)
      trace_ << "s " << unit << ' ' << want << ' ' << least << ' ' << multiple << ' '
             << max_pieces << ' ' << pieces.size() << '\n';
    return pieces;
  }
  size_t elastic(size_t want, size_t least) {
    if (least > want) least = want;
    std::lock_guard<std::mutex> lk(mu_);
    // Recorded so that a replay can make the same choice against its own
    // arena: the request that follows is the buffer sized by this answer.
    if (tracing_) trace_ << "e " << want << ' ' << least << '\n';
    return arena_.elastic_fit(want, least);
  }

  // Allocation history: every live block first (as allocated), then each
  // request and release in order.
  void history_start() {
    std::lock_guard<std::mutex> lk(mu_);
    trace_.str(std::string());
    trace_.clear();
    trace_ids_.clear();
    next_id_ = 0;
    tracing_ = true;
    for (const auto& [addr, size] : arena_live_snapshot()) {
      trace_ids_[addr] = next_id_;
      trace_ << "a " << next_id_++ << ' ' << size << '\n';
    }
  }
  void history_mark(const std::string& label) {
    std::lock_guard<std::mutex> lk(mu_);
    if (tracing_) trace_ << "m " << label << '\n';
  }
  void history_stop(const std::string& path) {
    std::lock_guard<std::mutex> lk(mu_);
    tracing_ = false;
    trace_ids_.clear();
    std::ofstream out(path);
    if (!out) throw std::runtime_error("allocation history: cannot write " + path);
    out << trace_.str();
    trace_.str(std::string());
  }

 private:
  std::vector<std::pair<uintptr_t, size_t>> arena_live_snapshot() { return arena_.live_blocks(); }
  void sample_locked() {
    size_t fr = 0, tot = 0;
    if (ember_mem_get_info(&fr, &tot) != EMBER_OK) return;
    device_used_ = tot - fr;
    peak_device_used_ = std::max(peak_device_used_, device_used_);
  }

  std::mutex mu_;
  HipBackend backend_;
  detail::BlockArena arena_;
  size_t high_water_ = 0;  // like the peak of live bytes, but never reset
  size_t device_used_ = 0, peak_device_used_ = 0;
  bool tracing_ = false;
  std::ostringstream trace_;
  std::unordered_map<uintptr_t, uint64_t> trace_ids_;
  uint64_t next_id_ = 0;
};

class CpuAllocator final : public Allocator {
 public:
  void* allocate(size_t nbytes) override {
    if (nbytes == 0) return nullptr;
    void* p = std::aligned_alloc(64, (nbytes + 63) & ~size_t{63});
    if (!p) throw std::runtime_error("cpu_allocator: out of memory");
    return p;
  }
  void deallocate(void* ptr) noexcept override { std::free(ptr); }
  Device device() const override { return kCPU; }
};

class PinnedCpuAllocator final : public Allocator {
 public:
  void* allocate(size_t nbytes) override {
    if (nbytes == 0) return nullptr;
    void* p = nullptr;
    runtime::check(ember_host_malloc_pinned(&p, nbytes), "pinned_cpu_allocator");
    std::lock_guard<std::mutex> lk(mu_);
    sizes_[p] = nbytes;
    bytes_ += nbytes;
    return p;
  }
  void deallocate(void* ptr) noexcept override {
    if (!ptr) return;
    {
      std::lock_guard<std::mutex> lk(mu_);
      auto it = sizes_.find(ptr);
      if (it != sizes_.end()) {
        bytes_ -= it->second;
        sizes_.erase(it);
      }
    }
    ember_host_free_pinned(ptr);
  }
  Device device() const override { return kCPU; }
  size_t bytes() {
    std::lock_guard<std::mutex> lk(mu_);
    return bytes_;
  }

 private:
  std::mutex mu_;
  std::unordered_map<void*, size_t> sizes_;
  size_t bytes_ = 0;
};

HipCachingAllocator& hip_cache() {
  static HipCachingAllocator* a = new HipCachingAllocator();  // outlives static tensors
  return *a;
}
PinnedCpuAllocator& pinned() {
  static PinnedCpuAllocator* a = new PinnedCpuAllocator();
  return *a;
}

}  // namespace

Allocator& hip_allocator() { return hip_cache(); }
Allocator& cpu_allocator() {
  static CpuAllocator a;
  return a;
}
Allocator& pinned_cpu_allocator() { return pinned(); }
Allocator& allocator_for(const Device& device) {
  return device.is_hip() ? hip_allocator() : cpu_allocator();
}

DeviceMemoryStats device_memory_stats() { return hip_cache().stats(); }
void reset_peak_device_memory() { hip_cache().reset_peak(); }
void empty_device_cache() { hip_cache().empty_cache(); }
void set_device_memory_limit(size_t bytes) { hip_cache().set_limit(bytes); }
void sample_device_memory() { hip_cache().sample(); }
std::vector<size_t> device_scatter_plan(size_t unit, size_t want, size_t least, size_t multiple,
                                        size_t max_pieces) {
  return hip_cache().scatter_plan(unit, want, least, multiple, max_pieces);
}
size_t elastic_workspace_bytes(size_t want, size_t least) {
  return hip_cache().elastic(want, least);
}
void start_allocation_history() { hip_cache().history_start(); }
void mark_allocation_history(const std::string& label) { hip_cache().history_mark(label); }
void stop_allocation_history(const std::string& path) { hip_cache().history_stop(path); }
size_t pinned_host_bytes() { return pinned().bytes(); }

// ------------------------------------------------------------------ Storage
Storage::Storage(size_t nbytes, Allocator& allocator)
    : allocator_(&allocator), nbytes_(nbytes), device_(allocator.device()) {
  data_ = allocator_->allocate(nbytes);
  pinned_ = (&allocator == &pinned_cpu_allocator());
}

Storage::Storage(Storage&& o) noexcept
    : allocator_(o.allocator_), data_(o.data_), nbytes_(o.nbytes_), device_(o.device_),
      pinned_(o.pinned_) {
  o.allocator_ = nullptr;
  o.data_ = nullptr;
  o.nbytes_ = 0;
}

Storage& Storage::operator=(Storage&& o) noexcept {
  if (this != &o) {
    release_();
    allocator_ = o.allocator_;
    data_ = o.data_;
    nbytes_ = o.nbytes_;
    device_ = o.device_;
    pinned_ = o.pinned_;
    o.allocator_ = nullptr;
    o.data_ = nullptr;
    o.nbytes_ = 0;
  }
  return *this;
}

Storage::~Storage() { release_(); }

void Storage::release_() noexcept {
  if (allocator_ && data_) allocator_->deallocate(data_);
  data_ = nullptr;
}

}  // namespace ctd
