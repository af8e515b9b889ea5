#pragma once
// safetensors file I/O (the reference's include/ctd/safetensors.h:14-20 keeps
// its two functions and their signatures; SafetensorsReader is added).
// The writer emits fp32 tensors with a compact, key-sorted JSON header padded
// with spaces to a multiple of 8 bytes and data in insertion order.

#include <cstdint>
#include <filesystem>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "ctd/tensor.h"

namespace ctd {

using TensorDict = std::unordered_map<std::string, Tensor>;

// Every tensor of the file, allocated on `device`.  Readable dtypes: F32, I64,
// I32.  Errors (unreadable file, malformed header, ranges outside the data
// region or overlapping, a size that does not match dtype x shape, another
// dtype) throw std::runtime_error before any tensor is allocated.
TensorDict load_safetensors(const std::filesystem::path& path, Device device);

void save_safetensors(const std::vector<std::pair<std::string, Tensor>>& named_tensors,
                      const std::filesystem::path& path);

// One file opened for random access: the header is parsed and the layout
// checked on construction (as load_safetensors does), and read() copies one
// tensor's bytes into memory the caller owns, e.g. a model parameter or a
// pinned optimizer-state buffer, without an intermediate tensor.
class SafetensorsReader {
 public:
  struct Entry {
    std::string name;
    DType dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;  // byte range within the data region
  };

  explicit SafetensorsReader(const std::filesystem::path& path);
  ~SafetensorsReader();
  SafetensorsReader(const SafetensorsReader&) = delete;
  SafetensorsReader& operator=(const SafetensorsReader&) = delete;

  // Entries in header order (the writer's header is key-sorted).
  const std::vector<Entry>& entries() const { return entries_; }
  // The entry called `name`, or nullptr.
  const Entry* find(const std::string& name) const;
  // Copies entry `name` into `dst`, which must have its dtype, shape and be
  // contiguous; a device tensor is filled through pinned staging buffers and
  // the copies are complete when read() returns.
  void read(const std::string& name, Tensor& dst) const;

 private:
  std::filesystem::path path_;
  int fd_ = -1;
  uint64_t data_origin_ = 0;
  std::vector<Entry> entries_;
  std::unordered_map<std::string, size_t> index_;

  friend TensorDict load_safetensors(const std::filesystem::path&, Device);
  void read_bytes(const Entry& e, void* dst, bool dst_on_device) const;
};

}  // namespace ctd
