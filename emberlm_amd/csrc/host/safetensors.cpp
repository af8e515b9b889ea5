// safetensors reader and writer over POSIX file descriptors.
//
// The file format (fixed by safetensors; the reference reads and writes it in
// src/core/safetensors.cpp): an 8-byte little-endian header length n, n bytes
// of JSON mapping each tensor name to {"data_offsets":[b,e],"dtype":...,
// "shape":[...]} (plus an optional "__metadata__" entry), then the data region
// those offsets index.
//
// Reading.  The header is parsed and the whole layout checked against the
// file's size before anything is allocated.  Host destinations are filled by
// pread in place; device destinations stream through a ring of two pinned
// buffers, so the disk read of one chunk overlaps the host-to-device copy of
// the one before (a 1.24 GB embedding is never staged whole in pageable
// memory).
//
// Writing.  The header must come out byte-identical to the reference writer's
// (nlohmann::json, whose objects are std::maps): keys sorted, each entry's
// fields in the order data_offsets, dtype, shape, no spaces, then spaces up
// to a multiple of 8 bytes; data in the caller's order.  Device tensors
// stream out through the same pinned ring (chunk k+1 is copied while chunk k
// is written).  The file is written under a temporary name and renamed into
// place, so an interrupted save leaves any previous file intact.
#include "ctd/safetensors.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ctd/runtime.h"
#include "json.h"

namespace ctd {

namespace {

enum class Fault { kIo, kTruncated, kHeader, kLayout, kDtype, kArgument };

[[noreturn]] void fault(Fault f, const std::filesystem::path& p, const std::string& detail) {
  static const char* const kWhat[] = {"I/O error", "truncated file", "malformed header",
                                      "inconsistent layout", "unsupported dtype",
                                      "invalid argument"};
  throw std::runtime_error("safetensors " + p.string() + ": " + kWhat[static_cast<int>(f)] +
                           ": " + detail);
}

// Reads exactly `n` bytes at `off` (pread moves at most ~2 GiB per call).
void pread_full(int fd, void* dst, uint64_t n, uint64_t off, const std::filesystem::path& p) {
  auto* d = static_cast<char*>(dst);
  while (n > 0) {
    const ssize_t got = ::pread(fd, d, static_cast<size_t>(std::min<uint64_t>(n, 1u << 30)),
                                static_cast<off_t>(off));
    if (got < 0 && errno == EINTR) continue;
    if (got < 0) fault(Fault::kIo, p, std::strerror(errno));
    if (got == 0) fault(Fault::kTruncated, p, "end of file inside a tensor");
    d += got;
    off += static_cast<uint64_t>(got);
    n -= static_cast<uint64_t>(got);
  }
}

void write_full(int fd, const void* src, uint64_t n, const std::filesystem::path& p) {
  const auto* s = static_cast<const char*>(src);
  while (n > 0) {
    const ssize_t put = ::write(fd, s, static_cast<size_t>(std::min<uint64_t>(n, 1u << 30)));
    if (put < 0 && errno == EINTR) continue;
    if (put <= 0) fault(Fault::kIo, p, std::strerror(errno));
    s += put;
    n -= static_cast<uint64_t>(put);
  }
}

// A non-negative JSON integer (the parser keeps a number's source text).
uint64_t json_uint(const json::JVal& v, const std::filesystem::path& p, const char* what) {
  if (v.kind != json::JVal::kNum || v.str.empty() ||
      v.str.find_first_not_of("0123456789") != std::string::npos)
    fault(Fault::kHeader, p, std::string(what) + " is not a non-negative integer");
  return std::stoull(v.str);
}

bool readable_dtype(const std::string& s, DType* out) {
  if (s == "F32") *out = DType::kFloat32;
  else if (s == "I64") *out = DType::kInt64;
  else if (s == "I32") *out = DType::kInt32;
  else return false;
  return true;
}

// Two pinned host buffers with one event each: the host fills (or drains) one
// while the stream copies the other.
class StagingRing {
 public:
  static constexpr size_t kSlotBytes = size_t{64} << 20;

  explicit StagingRing(size_t largest) : bytes_(std::max<size_t>(1, std::min(largest, kSlotBytes))) {
    for (Slot& s : slots_) {
      CTD_CHECK(ember_host_malloc_pinned(&s.buf, bytes_));
      CTD_CHECK(ember_event_create(&s.copied));
    }
  }
  ~StagingRing() {
    for (Slot& s : slots_) {
      if (s.copied) {
        ember_event_synchronize(s.copied);
        ember_event_destroy(s.copied);
      }
      if (s.buf) ember_host_free_pinned(s.buf);
    }
  }
  StagingRing(const StagingRing&) = delete;
  StagingRing& operator=(const StagingRing&) = delete;

  size_t slot_bytes() const { return bytes_; }
  // Buffer k % 2, once the copy last issued on it has finished.
  void* acquire(uint64_t k) {
    Slot& s = slots_[k & 1];
    CTD_CHECK(ember_event_synchronize(s.copied));
    return s.buf;
  }
  void* peek(uint64_t k) { return slots_[k & 1].buf; }
  void issued(uint64_t k, ember_stream_t st) { CTD_CHECK(ember_event_record(slots_[k & 1].copied, st)); }
  void drain() {
    for (Slot& s : slots_) CTD_CHECK(ember_event_synchronize(s.copied));
  }

 private:
  struct Slot {
    void* buf = nullptr;
    ember_event_t copied = nullptr;
  };
  size_t bytes_;
  Slot slots_[2];
};

}  // namespace

// ------------------------------------------------------------------ reading

SafetensorsReader::SafetensorsReader(const std::filesystem::path& path) : path_(path) {
  fd_ = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd_ < 0) fault(Fault::kIo, path, std::string("cannot open: ") + std::strerror(errno));
  struct stat st {};
  if (::fstat(fd_, &st) != 0) {
    ::close(fd_);
    fault(Fault::kIo, path, std::strerror(errno));
  }
  try {
    const uint64_t file_bytes = static_cast<uint64_t>(st.st_size);
    if (file_bytes < 8) fault(Fault::kTruncated, path, "no header length");
    uint64_t n = 0;
    pread_full(fd_, &n, 8, 0, path);
    if (n > file_bytes - 8) fault(Fault::kTruncated, path, "header runs past the end of the file");
    if (n > (uint64_t{1} << 30)) fault(Fault::kHeader, path, "header longer than 1 GiB");
    std::string text(n, '\0');
    pread_full(fd_, text.data(), n, 8, path);
    const json::JVal top = json::Parser(text, "safetensors " + path.string() + ": malformed header").parse();
    if (top.kind != json::JVal::kObj) fault(Fault::kHeader, path, "not a JSON object");
    data_origin_ = 8 + n;
    const uint64_t data_bytes = file_bytes - data_origin_;

    for (const auto& [name, spec] : top.obj) {
      if (name == "__metadata__") continue;
      if (spec.kind != json::JVal::kObj) fault(Fault::kHeader, path, name + " is not an object");
      const json::JVal* dt = spec.find("dtype");
      const json::JVal* sh = spec.find("shape");
      const json::JVal* of = spec.find("data_offsets");
      if (!dt || dt->kind != json::JVal::kStr || !sh || sh->kind != json::JVal::kArr || !of ||
          of->kind != json::JVal::kArr || of->arr.size() != 2)
        fault(Fault::kHeader, path, name + " needs dtype, shape and two data_offsets");
      Entry e;
      e.name = name;
      if (!readable_dtype(dt->str, &e.dtype))
        fault(Fault::kDtype, path, name + " is " + dt->str + " (readable: F32, I64, I32)");
      // Element and byte counts are formed without wrapping: a shape whose
      // product passes 2^63 cannot describe bytes of this file.
      uint64_t count = 1;
      bool too_big = false;
      for (const json::JVal& d : sh->arr) {
        const uint64_t extent = json_uint(d, path, "a shape extent");
        too_big = too_big || extent > static_cast<uint64_t>(INT64_MAX) ||
                  __builtin_mul_overflow(count, extent, &count);
        e.shape.push_back(static_cast<int64_t>(extent));
      }
      uint64_t need = 0;
      too_big = too_big || __builtin_mul_overflow(count, static_cast<uint64_t>(dtype_size(e.dtype)),
                                                  &need) ||
                need > static_cast<uint64_t>(INT64_MAX);
      if (too_big) fault(Fault::kLayout, path, name + " has a shape too large to address");
      e.begin = json_uint(of->arr[0], path, "a data offset");
      e.end = json_uint(of->arr[1], path, "a data offset");
      if (e.end < e.begin || e.end > data_bytes)
        fault(Fault::kLayout, path, name + " lies outside the data region");
      if (e.end - e.begin != need)
        fault(Fault::kLayout, path, name + " holds " + std::to_string(e.end - e.begin) +
                                        " bytes, its dtype and shape need " +
                                        std::to_string(need));
      index_.emplace(name, entries_.size());
      entries_.push_back(std::move(e));
    }
    // No two tensors may share bytes.
    std::vector<const Entry*> by_offset;
    for (const Entry& e : entries_)
      if (e.end > e.begin) by_offset.push_back(&e);
    std::sort(by_offset.begin(), by_offset.end(),
              [](const Entry* a, const Entry* b) { return a->begin < b->begin; });
    for (size_t i = 1; i < by_offset.size(); ++i)
      if (by_offset[i]->begin < by_offset[i - 1]->end)
        fault(Fault::kLayout, path, by_offset[i - 1]->name + " and " + by_offset[i]->name +
                                        " overlap");
  } catch (...) {
    ::close(fd_);
    fd_ = -1;
    throw;
  }
}

SafetensorsReader::~SafetensorsReader() {
  if (fd_ >= 0) ::close(fd_);
}

const SafetensorsReader::Entry* SafetensorsReader::find(const std::string& name) const {
  auto it = index_.find(name);
  return it == index_.end() ? nullptr : &entries_[it->second];
}

void SafetensorsReader::read_bytes(const Entry& e, void* dst, bool dst_on_device) const {
  const uint64_t n = e.end - e.begin;
  if (n == 0) return;
  if (!dst_on_device) {
    pread_full(fd_, dst, n, data_origin_ + e.begin, path_);
    return;
  }
  StagingRing ring(static_cast<size_t>(n));
  const ember_stream_t st = runtime::compute_stream();
  const uint64_t slot = ring.slot_bytes();
  for (uint64_t k = 0, off = 0; off < n; ++k, off += slot) {
    const uint64_t len = std::min(slot, n - off);
    void* buf = ring.acquire(k);
    pread_full(fd_, buf, len, data_origin_ + e.begin + off, path_);
    CTD_CHECK(ember_memcpy_async(static_cast<char*>(dst) + off, buf, len, 0, st));
    ring.issued(k, st);
  }
  ring.drain();
}

void SafetensorsReader::read(const std::string& name, Tensor& dst) const {
  const Entry* e = find(name);
  if (!e) fault(Fault::kArgument, path_, "no tensor named " + name);
  if (dst.dtype() != e->dtype || dst.shape() != e->shape || !dst.is_contiguous())
    fault(Fault::kArgument, path_, name + ": destination differs in dtype, shape or layout");
  read_bytes(*e, dst.data_ptr(), dst.device().is_hip());
}

TensorDict load_safetensors(const std::filesystem::path& path, Device device) {
  const SafetensorsReader r(path);
  TensorDict out;
  for (const SafetensorsReader::Entry& e : r.entries()) {
    Tensor t = Tensor::empty(e.shape, e.dtype, device);
    r.read_bytes(e, t.data_ptr(), device.is_hip());
    out.emplace(e.name, std::move(t));
  }
  return out;
}

// ------------------------------------------------------------------ writing

void save_safetensors(const std::vector<std::pair<std::string, Tensor>>& named_tensors,
                      const std::filesystem::path& path) {
  // Header: name -> entry text, the map's order being the sorted key order.
  std::map<std::string, std::string> fields;
  uint64_t at = 0;
  size_t largest_device = 0;
  for (const auto& [name, t] : named_tensors) {
    if (t.dtype() != DType::kFloat32)
      fault(Fault::kArgument, path, name + ": the writer stores F32 tensors only");
    if (!t.is_contiguous()) fault(Fault::kArgument, path, name + " is not contiguous");
    if (fields.count(name) != 0) fault(Fault::kArgument, path, name + " appears twice");
    std::string f = "{\"data_offsets\":[" + std::to_string(at) + "," +
                    std::to_string(at + t.nbytes()) + "],\"dtype\":\"F32\",\"shape\":[";
    for (size_t i = 0; i < t.shape().size(); ++i)
      f += (i ? "," : "") + std::to_string(t.shape()[i]);
    f += "]}";
    fields.emplace(name, std::move(f));
    at += t.nbytes();
    if (t.device().is_hip()) largest_device = std::max(largest_device, t.nbytes());
  }
  std::string header = "{";
  for (const auto& [name, f] : fields) {
    if (header.size() > 1) header += ',';
    json::append_quoted(header, name);
    header += ':';
    header += f;
  }
  header += '}';
  header.append((8 - header.size() % 8) % 8, ' ');

  const std::filesystem::path tmp = path.string() + ".partial";
  const int fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
  if (fd < 0) fault(Fault::kIo, tmp, std::string("cannot create: ") + std::strerror(errno));
  try {
    const uint64_t n = header.size();
    write_full(fd, &n, 8, tmp);
    write_full(fd, header.data(), n, tmp);
    std::unique_ptr<StagingRing> ring;
    if (largest_device > 0) ring = std::make_unique<StagingRing>(largest_device);
    const ember_stream_t st = largest_device > 0 ? runtime::compute_stream() : nullptr;
    for (const auto& [name, t] : named_tensors) {
      const uint64_t bytes = t.nbytes();
      if (bytes == 0) continue;
      if (!t.device().is_hip()) {
        write_full(fd, t.data_ptr(), bytes, tmp);
        continue;
      }
      const char* src = static_cast<const char*>(t.data_ptr());
      const uint64_t slot = ring->slot_bytes();
      const uint64_t chunks = (bytes + slot - 1) / slot;
      auto issue = [&](uint64_t k) {
        void* buf = ring->acquire(k);
        CTD_CHECK(ember_memcpy_async(buf, src + k * slot, std::min(slot, bytes - k * slot), 1, st));
        ring->issued(k, st);
      };
      issue(0);
      for (uint64_t k = 0; k < chunks; ++k) {
        if (k + 1 < chunks) issue(k + 1);
        ring->acquire(k);  // chunk k has arrived
        write_full(fd, ring->peek(k), std::min(slot, bytes - k * slot), tmp);
      }
    }
  } catch (...) {
    ::close(fd);
    ::unlink(tmp.c_str());
    throw;
  }
  if (::close(fd) != 0) fault(Fault::kIo, tmp, std::strerror(errno));
  std::error_code ec;
  std::filesystem::rename(tmp, path, ec);
  if (ec) fault(Fault::kIo, path, "cannot move the written file into place: " + ec.message());
}

}  // namespace ctd
