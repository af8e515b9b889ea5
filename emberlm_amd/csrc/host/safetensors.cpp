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

namespace ctd {

namespace {

struct FileCloser {
  void operator()(std::FILE* f) const noexcept {
    if (f) std::fclose(f);
  }
};
using FilePtr = std::unique_ptr<std::FILE, FileCloser>;

// ---- minimal JSON value / parser (objects, arrays, strings, numbers, literals)
struct JVal {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  double num = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;
  const JVal& at(const std::string& k) const {
    for (const auto& [key, v] : obj)
      if (key == k) return v;
    throw std::runtime_error("safetensors: header entry missing '" + k + "'");
  }
};

class Parser {
 public:
  explicit Parser(const std::string& s) : s_(s) {}
  JVal parse() {
    JVal v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* m) {
    throw std::runtime_error(std::string("safetensors: bad header JSON (") + m + ") at byte " +
                             std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\t' || s_[i_] == '\r'))
      ++i_;
  }
  char peek() {
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    return s_[i_];
  }
  void expect(char c) {
    if (peek() != c) fail("unexpected character");
    ++i_;
  }
  JVal value() {
    const char c = peek();
    if (c == '{') return object();
    if (c == '[') return array();
    if (c == '"') {
      JVal v;
      v.kind = JVal::kStr;
      v.str = string();
      return v;
    }
    if (c == 't' || c == 'f' || c == 'n') return literal();
    return number();
  }
  JVal object() {
    JVal v;
    v.kind = JVal::kObj;
    expect('{');
    if (peek() == '}') {
      ++i_;
      return v;
    }
    for (;;) {
      std::string k = string();
      expect(':');
      v.obj.emplace_back(std::move(k), value());
      const char c = peek();
      ++i_;
      if (c == '}') break;
      if (c != ',') fail("expected , or }");
    }
    return v;
  }
  JVal array() {
    JVal v;
    v.kind = JVal::kArr;
    expect('[');
    if (peek() == ']') {
      ++i_;
      return v;
    }
    for (;;) {
      v.arr.push_back(value());
      const char c = peek();
      ++i_;
      if (c == ']') break;
      if (c != ',') fail("expected , or ]");
    }
    return v;
  }
  std::string string() {
    expect('"');
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c == '\\') {
        if (i_ >= s_.size()) fail("bad escape");
        const char e = s_[i_++];
        switch (e) {
          case 'n': out += '\n'; break;
          case 't': out += '\t'; break;
          case 'r': out += '\r'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'u': {
            if (i_ + 4 > s_.size()) fail("bad \\u escape");
            const unsigned cp = static_cast<unsigned>(std::stoul(s_.substr(i_, 4), nullptr, 16));
            i_ += 4;
            if (cp < 0x80) {
              out += static_cast<char>(cp);
            } else if (cp < 0x800) {
              out += static_cast<char>(0xC0 | (cp >> 6));
              out += static_cast<char>(0x80 | (cp & 0x3F));
            } else {
              out += static_cast<char>(0xE0 | (cp >> 12));
              out += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
              out += static_cast<char>(0x80 | (cp & 0x3F));
            }
            break;
          }
          default: out += e;
        }
      } else {
        out += c;
      }
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  JVal number() {
    const size_t b = i_;
    while (i_ < s_.size() && (std::strchr("+-0123456789.eE", s_[i_]) != nullptr)) ++i_;
    if (b == i_) fail("expected a value");
    JVal v;
    v.kind = JVal::kNum;
    v.num = std::stod(s_.substr(b, i_ - b));
    v.str = s_.substr(b, i_ - b);
    return v;
  }
  JVal literal() {
    JVal v;
    if (s_.compare(i_, 4, "true") == 0) {
      v.kind = JVal::kBool;
      v.num = 1;
      i_ += 4;
    } else if (s_.compare(i_, 5, "false") == 0) {
      v.kind = JVal::kBool;
      i_ += 5;
    } else if (s_.compare(i_, 4, "null") == 0) {
      i_ += 4;
    } else {
      fail("bad literal");
    }
    return v;
  }
  const std::string& s_;
  size_t i_ = 0;
};

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
  const JVal json = Parser(header).parse();
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
