// safetensors reader/writer.
//
// Reference: src/core/safetensors.cpp (nlohmann::json).  The format is: u64
// little-endian header length, a JSON object {name: {"dtype", "shape",
// "data_offsets"}} (plus an optional "__metadata__" of strings), then the raw
// data.  The writer reproduces the reference's bytes: the header is the compact
// JSON dump of a key-sorted object (nlohmann's object is a std::map), entries
// in key order "data_offsets", "dtype", "shape", padded with spaces to a
// multiple of 8, and tensor data in insertion order.  The reader accepts F32,
// I64 and I32 like the reference.  A small JSON parser is built in because
// no JSON library is available offline.
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ctd/runtime.h"
#include "ctd/safetensors.h"
#include "json.h"

namespace ctd {

namespace {

struct FileCloser {
  void operator()(std::FILE* f) const noexcept {
    if (f) std::fclose(f);
  }
};
using FilePtr = std::unique_ptr<std::FILE, FileCloser>;

using json::JVal;

JVal parse_header(const std::string& text) { return json::Parser(text, "safetensors: bad header JSON").parse(); }

uint64_t as_u64(const JVal& v) {
  if (v.kind != JVal::kNum) throw std::runtime_error("safetensors: expected an integer");
  return std::stoull(v.str);
}

DType parse_dtype(const std::string& s) {
  if (s == "F32") return DType::kFloat32;
  if (s == "F16") return DType::kFloat16;
  if (s == "BF16") return DType::kBFloat16;
  if (s == "I64") return DType::kInt64;
  if (s == "I32") return DType::kInt32;
  throw std::runtime_error("safetensors: unsupported dtype '" + s + "'");
}

void json_escape(std::string& out, const std::string& s) {
  out += '"';
  for (unsigned char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\n': out += "\\n"; break;
      case '\t': out += "\\t"; break;
      case '\r': out += "\\r"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof buf, "\\u%04x", c);
          out += buf;
        } else {
          out += static_cast<char>(c);
        }
    }
  }
  out += '"';
}

}  // namespace

TensorDict load_safetensors(const std::filesystem::path& path, Device device) {
  FilePtr fp(std::fopen(path.c_str(), "rb"));
  if (!fp) throw std::runtime_error("safetensors: cannot open " + path.string());
  uint64_t header_size = 0;
  if (std::fread(&header_size, sizeof(header_size), 1, fp.get()) != 1)
    throw std::runtime_error("safetensors: short read on header length");
  if (header_size > (uint64_t{1} << 30)) throw std::runtime_error("safetensors: header too large");
  std::string header(header_size, '\0');
  if (std::fread(header.data(), 1, header_size, fp.get()) != header_size)
    throw std::runtime_error("safetensors: short read on header");
  const JVal json = parse_header(header);
  if (json.kind != JVal::kObj) throw std::runtime_error("safetensors: header is not an object");
  const int64_t data_origin = static_cast<int64_t>(8 + header_size);

  TensorDict out;
  std::vector<uint8_t> staging;
  for (const auto& [name, spec] : json.obj) {
    if (name == "__metadata__") continue;
    const std::string dtype_str = spec.at("dtype").str;
    const DType dtype = parse_dtype(dtype_str);
    if (dtype != DType::kFloat32 && dtype != DType::kInt64 && dtype != DType::kInt32)
      throw std::runtime_error("safetensors: " + name + " has dtype " + dtype_str +
                               " which is not supported on the read path");
    std::vector<int64_t> shape;
    for (const auto& d : spec.at("shape").arr) shape.push_back(static_cast<int64_t>(as_u64(d)));
    const auto& offs = spec.at("data_offsets").arr;
    if (offs.size() != 2) throw std::runtime_error("safetensors: bad data_offsets");
    const uint64_t b = as_u64(offs[0]), e = as_u64(offs[1]);
    if (e < b) throw std::runtime_error("safetensors: bad data_offsets");
    const uint64_t nbytes = e - b;
    Tensor t = Tensor::empty(shape, dtype, device);
    if (t.nbytes() != nbytes) throw std::runtime_error("safetensors: size mismatch for " + name);
    if (nbytes == 0) {
      out.emplace(name, std::move(t));
      continue;
    }
    void* dst = t.data_ptr();
    if (device.is_hip()) {
      staging.resize(nbytes);
      dst = staging.data();
    }
    if (std::fseek(fp.get(), static_cast<long>(data_origin + static_cast<int64_t>(b)), SEEK_SET) != 0)
      throw std::runtime_error("safetensors: seek failed for " + name);
    if (std::fread(dst, 1, nbytes, fp.get()) != nbytes)
      throw std::runtime_error("safetensors: short read for tensor " + name);
    if (device.is_hip()) {
      CTD_CHECK(ember_memcpy_async(t.data_ptr(), staging.data(), nbytes, 0,
                                   runtime::compute_stream()));
      runtime::synchronize();
    }
    out.emplace(name, std::move(t));
  }
  return out;
}

void save_safetensors(const std::vector<std::pair<std::string, Tensor>>& named_tensors,
                      const std::filesystem::path& path) {
  // name -> serialized entry, key-sorted like nlohmann::json's std::map object.
  std::map<std::string, std::string> entries;
  uint64_t running = 0;
  for (const auto& [name, t] : named_tensors) {
    if (t.dtype() != DType::kFloat32)
      throw std::runtime_error("save_safetensors: only fp32 supported, got " + name);
    if (!t.is_contiguous()) throw std::runtime_error("save_safetensors: non-contiguous tensor " + name);
    std::string e = "{\"data_offsets\":[" + std::to_string(running) + "," +
                    std::to_string(running + t.nbytes()) + "],\"dtype\":\"F32\",\"shape\":[";
    for (size_t i = 0; i < t.shape().size(); ++i) {
      if (i) e += ",";
      e += std::to_string(t.shape()[i]);
    }
    e += "]}";
    entries[name] = std::move(e);
    running += t.nbytes();
  }
  std::string header = "{";
  bool first = true;
  for (const auto& [name, e] : entries) {
    if (!first) header += ",";
    first = false;
    json_escape(header, name);
    header += ":";
    header += e;
  }
  header += "}";
  while (header.size() % 8 != 0) header.push_back(' ');
  const uint64_t header_size = header.size();

  FilePtr fp(std::fopen(path.c_str(), "wb"));
  if (!fp) throw std::runtime_error("save_safetensors: cannot open " + path.string());
  if (std::fwrite(&header_size, sizeof(header_size), 1, fp.get()) != 1)
    throw std::runtime_error("save_safetensors: short write on header size");
  if (std::fwrite(header.data(), 1, header.size(), fp.get()) != header.size())
    throw std::runtime_error("save_safetensors: short write on header");
  std::vector<uint8_t> staging;
  for (const auto& [name, t] : named_tensors) {
    const size_t nb = t.nbytes();
    if (nb == 0) continue;
    const void* src = t.data_ptr();
    if (t.device().is_hip()) {
      staging.resize(nb);
      t.copy_to_host(staging.data());
      src = staging.data();
    }
    if (std::fwrite(src, 1, nb, fp.get()) != nb)
      throw std::runtime_error("save_safetensors: short write for tensor " + name);
  }
}

}  // namespace ctd
