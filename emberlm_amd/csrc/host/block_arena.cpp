// BlockArena: best-fit placement with splitting and coalescing (see the header).
#include "block_arena.h"

#include <algorithm>
#include <fstream>
#include <sstream>
#include <stdexcept>

namespace ctd::detail {

BlockArena::~BlockArena() {
  // Blocks and segment records only; the memory itself is the backend's (the
  // process-wide device allocator is never destroyed).
  std::vector<Block*> all;
  for (Block* b : free_small_) all.push_back(b);
  for (Block* b : free_large_) all.push_back(b);
  for (auto& [a, b] : live_) all.push_back(b);
  for (Block* b : all) delete b;
  for (Segment* s : segments_) delete s;
}

BlockArena::Block* BlockArena::take_fit(FreeSet& set, size_t size) {
  Block key{0, size, nullptr, nullptr, nullptr, true};
  auto it = set.lower_bound(&key);  // smallest size >= request, lowest address first
  if (it == set.end()) return nullptr;
  Block* b = *it;
  set.erase(it);
  return b;
}

BlockArena::Block* BlockArena::grow(bool small, size_t size) {
  const size_t seg_bytes =
      small ? kSmallSegment
            : (size + kLargeSegmentGranule - 1) / kLargeSegmentGranule * kLargeSegmentGranule;
  if (limit_ && stats_.held_bytes + seg_bytes > limit_) return nullptr;
  uintptr_t base = 0;
  if (!backend_.obtain(seg_bytes, &base)) return nullptr;
  auto* seg = new Segment{base, seg_bytes, small};
  segments_.push_back(seg);
  stats_.held_bytes += seg_bytes;
  stats_.peak_held_bytes = std::max(stats_.peak_held_bytes, stats_.held_bytes);
  stats_.segments_obtained += 1;
  stats_.segments += 1;
  return new Block{base, seg_bytes, seg, nullptr, nullptr, true};
}

// Marks the first `size` bytes of free block b as handed out; the rest stays
// a free block of its own.
BlockArena::Block* BlockArena::carve(Block* b, size_t size) {
  if (b->size > size) {
    auto* rest = new Block{b->addr + size, b->size - size, b->seg, b, b->hi, true};
    if (b->hi) b->hi->lo = rest;
    b->hi = rest;
    b->size = size;
    pool(b->seg->small).insert(rest);
  }
  b->free = false;
  b->seg->live += 1;
  live_[b->addr] = b;
  stats_.live_bytes += b->size;
  stats_.peak_live_bytes = std::max(stats_.peak_live_bytes, stats_.live_bytes);
  return b;
}

uintptr_t BlockArena::allocate(size_t bytes) {
  if (bytes == 0) throw std::runtime_error("BlockArena: zero-byte request");
  const size_t size = round_request(bytes);
  const bool small = size <= kSmallRequest;
  FreeSet& set = pool(small);
  Block* b = take_fit(set, size);
  if (!b) b = grow(small, size);
  if (!b) {
    // Nothing cached fits and the backend (or the limit) refuses a new
    // segment: give the wholly free segments back and try once more.
    stats_.trims += 1;
    give_back_free_segments();
    b = take_fit(set, size);
    if (!b) b = grow(small, size);
  }
  if (!b)
    throw std::runtime_error(
        "device allocator: out of memory for " + std::to_string(bytes) + " bytes (held " +
        std::to_string(stats_.held_bytes) + ", live " + std::to_string(stats_.live_bytes) +
        (limit_ ? ", limit " + std::to_string(limit_) : std::string()) + ")");
  return carve(b, size)->addr;
}

size_t BlockArena::release(uintptr_t addr) {
  auto it = live_.find(addr);
  if (it == live_.end()) return 0;
  Block* b = it->second;
  live_.erase(it);
  const size_t size = b->size;
  stats_.live_bytes -= size;
  b->seg->live -= 1;
  b->free = true;
  FreeSet& set = pool(b->seg->small);
  // Merge with the free neighbour above, then with the one below.
  if (Block* h = b->hi; h && h->free) {
    set.erase(h);
    b->size += h->size;
    b->hi = h->hi;
    if (h->hi) h->hi->lo = b;
    delete h;
  }
  if (Block* l = b->lo; l && l->free) {
    set.erase(l);
    l->size += b->size;
    l->hi = b->hi;
    if (b->hi) b->hi->lo = l;
    delete b;
    b = l;
  }
  set.insert(b);
  return size;
}

void BlockArena::give_back_free_segments() {
  bool any = false;
  for (Segment* s : segments_) any = any || s->live == 0;
  if (!any) return;
  backend_.quiesce();
  std::vector<Segment*> keep;
  for (Segment* s : segments_) {
    if (s->live != 0) {
      keep.push_back(s);
      continue;
    }
    // A segment without live blocks is one free block spanning all of it.
    FreeSet& set = pool(s->small);
    for (auto it = set.begin(); it != set.end();) {
      if ((*it)->seg == s) {
        delete *it;
        it = set.erase(it);
      } else {
        ++it;
      }
    }
    backend_.give_back(s->base, s->size);
    stats_.held_bytes -= s->size;
    stats_.segments -= 1;
    delete s;
  }
  segments_.swap(keep);
}

void BlockArena::trim() { give_back_free_segments(); }

size_t BlockArena::largest_free() const {
  size_t m = 0;
  if (!free_large_.empty()) m = (*free_large_.rbegin())->size;
  if (!free_small_.empty()) m = std::max(m, (*free_small_.rbegin())->size);
  return m;
}

bool BlockArena::fits(size_t bytes) const {
  const size_t size = round_request(bytes);
  const FreeSet& set = size <= kSmallRequest ? free_small_ : free_large_;
  return !set.empty() && (*set.rbegin())->size >= size;
}

std::vector<size_t> BlockArena::scatter_fit(size_t unit, size_t want, size_t least,
                                            size_t multiple, size_t max_pieces) const {
  std::vector<size_t> pieces;
  if (unit == 0 || want == 0 || max_pieces == 0) return pieces;
  least = std::min(least, want);
  size_t placed = 0;
  // Descending piece sizes, each no larger than the block it was sized for:
  // served in this order, best fit puts every piece in some free block.
  for (auto it = free_large_.rbegin();
       it != free_large_.rend() && placed < want && pieces.size() + 1 < max_pieces; ++it) {
    size_t n = std::min((*it)->size / unit, want - placed);
    while (n > 0 && round_request(n * unit) > (*it)->size) --n;
    if (n == 0) break;  // the rest are smaller still
    pieces.push_back(n * unit);
    placed += n;
  }
  if (placed < least) {  // grow by no more than `least` needs
    pieces.push_back((least - placed) * unit);
    return pieces;
  }
  if (multiple > 1 && placed < want && placed >= multiple) {
    size_t cut = placed % multiple;  // taken off the smallest pieces
    while (cut > 0) {
      const size_t last = pieces.back() / unit;
      if (last <= cut) {
        pieces.pop_back();
        cut -= last;
      } else {
        pieces.back() -= cut * unit;
        cut = 0;
      }
    }
  }
  return pieces;
}

std::vector<std::pair<uintptr_t, size_t>> BlockArena::live_blocks() const {
  std::vector<std::pair<uintptr_t, size_t>> out;
  out.reserve(live_.size());
  for (const auto& [a, b] : live_) out.emplace_back(a, b->size);
  std::sort(out.begin(), out.end());
  return out;
}

namespace {
// Addresses only: segments never overlap and are never touched.
class CountingBackend final : public ArenaBackend {
 public:
  bool obtain(size_t bytes, uintptr_t* base) override {
    *base = next_;
    next_ += (bytes + 4095) / 4096 * 4096 + 4096;
    return true;
  }
  void give_back(uintptr_t, size_t) override {}
  void quiesce() override {}

 private:
  uintptr_t next_ = uintptr_t{1} << 40;
};
}  // namespace

ArenaStats replay_history(const std::string& path, size_t limit) {
  std::ifstream in(path);
  if (!in) throw std::runtime_error("replay_history: cannot open " + path);
  CountingBackend backend;
  BlockArena arena(backend);
  arena.set_limit(limit);
  std::unordered_map<uint64_t, uintptr_t> ids;
  std::string line;
  int64_t lineno = 0;
  uint64_t elastic_bytes = 0;  // nonzero: the next request's size (from an "e" record)
  uint64_t split_pending = 0;  // recorded pieces of a split workspace still to come
  std::vector<uintptr_t> split_blocks;
  std::unordered_map<uint64_t, std::vector<uintptr_t>> groups;
  while (std::getline(in, line)) {
    ++lineno;
    if (line.empty()) continue;
    std::istringstream ls(line);
    char op = 0;
    ls >> op;
    if (op == 'm') continue;
    if (op == 's') {
      // a split workspace: the replay plans its own pieces and allocates
      // them now; the recorded pieces (the next `count` requests) map to
      // them, all released with the first
      uint64_t unit = 0, want = 0, least = 0, multiple = 0, maxp = 0, count = 0;
      ls >> unit >> want >> least >> multiple >> maxp >> count;
      if (!ls || unit == 0 || want == 0)
        throw std::runtime_error("replay_history: bad split record at line " +
                                 std::to_string(lineno));
      std::vector<uintptr_t> got;
      for (size_t b : arena.scatter_fit(unit, want, least, multiple, maxp)) got.push_back(arena.allocate(b));
      split_pending = count;
      split_blocks = std::move(got);
      continue;
    }
    if (op == 'e') {
      uint64_t want = 0, least = 0;
      ls >> want >> least;
      if (!ls || want == 0)
        throw std::runtime_error("replay_history: bad elastic record at line " +
                                 std::to_string(lineno));
      elastic_bytes = arena.elastic_fit(want, std::min(least, want));
      continue;
    }
    uint64_t id = 0;
    ls >> id;
    if (!ls) throw std::runtime_error("replay_history: bad line " + std::to_string(lineno));
    if (op == 'a') {
      uint64_t bytes = 0;
      ls >> bytes;
      if (!ls || bytes == 0)
        throw std::runtime_error("replay_history: bad size at line " + std::to_string(lineno));
      if (ids.count(id))
        throw std::runtime_error("replay_history: id allocated twice at line " +
                                 std::to_string(lineno));
      if (split_pending) {
        --split_pending;
        groups[id] = std::move(split_blocks);
        split_blocks.clear();
        ids[id] = 0;
        continue;
      }
      if (elastic_bytes) bytes = elastic_bytes;
      elastic_bytes = 0;
      ids[id] = arena.allocate(bytes);
    } else if (op == 'f') {
      auto it = ids.find(id);
      if (it == ids.end())
        throw std::runtime_error("replay_history: free of unknown id at line " +
                                 std::to_string(lineno));
      auto g = groups.find(id);
      if (g != groups.end()) {
        for (uintptr_t a : g->second) arena.release(a);
        groups.erase(g);
      } else {
        arena.release(it->second);
      }
      ids.erase(it);
    } else {
      throw std::runtime_error("replay_history: unknown record at line " + std::to_string(lineno));
    }
  }
  return arena.stats();
}

}  // namespace ctd::detail
