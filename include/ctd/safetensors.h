#pragma once
// safetensors file I/O (mirrors include/ctd/safetensors.h of the reference).
// The writer emits fp32 tensors with a compact, key-sorted JSON header padded
// with spaces to a multiple of 8 bytes and data in insertion order.

#include <filesystem>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "ctd/tensor.h"

namespace ctd {

using TensorDict = std::unordered_map<std::string, Tensor>;

TensorDict load_safetensors(const std::filesystem::path& path, Device device);

void save_safetensors(const std::vector<std::pair<std::string, Tensor>>& named_tensors,
                      const std::filesystem::path& path);

}  // namespace ctd
