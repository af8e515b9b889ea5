#pragma once
// Minimal JSON reader and writer for the host layer: safetensors headers and
// the training driver's config and loss log.  Objects keep their key order;
// numbers keep their source text so integers round-trip exactly.
#include <charconv>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace ctd::json {

struct JVal {
  enum Kind { kNull, kBool, kNum, kStr, kArr, kObj } kind = kNull;
  double num = 0;
  std::string str;
  std::vector<JVal> arr;
  std::vector<std::pair<std::string, JVal>> obj;

  const JVal* find(const std::string& k) const {
    for (const auto& [key, v] : obj)
      if (key == k) return &v;
    return nullptr;
  }
  const JVal& at(const std::string& k) const {
    if (const JVal* v = find(k)) return *v;
    throw std::runtime_error("JSON: entry missing '" + k + "'");
  }
};

class Parser {
 public:
  // `what` prefixes every error message, e.g. "safetensors: bad header JSON".
  Parser(const std::string& s, std::string what) : s_(s), what_(std::move(what)) {}
  JVal parse() {
    JVal v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  [[noreturn]] void fail(const char* m) {
    throw std::runtime_error(what_ + " (" + m + ") at byte " + std::to_string(i_));
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
  std::string what_;
  size_t i_ = 0;
};

// Shortest decimal text that reads back as the same double; integral values
// keep a ".0" so the field still reads as a floating-point number.
inline std::string number_text(double v) {
  char buf[64];
  auto [end, ec] = std::to_chars(buf, buf + sizeof(buf), v);
  if (ec != std::errc()) return "null";
  std::string s(buf, end);
  if (s.find_first_of(".eEn") == std::string::npos) s += ".0";  // n: inf/nan
  if (s == "inf" || s == "-inf" || s == "nan" || s == "-nan") return "null";
  return s;
}

// Appends s as a JSON string literal: quotes, backslashes and the short
// control escapes, other control bytes as \u00XX, everything else verbatim.
inline void append_quoted(std::string& out, const std::string& s) {
  out += '"';
  for (char c : s) {
    switch (c) {
      case '"': out += "\\\""; break;
      case '\\': out += "\\\\"; break;
      case '\b': out += "\\b"; break;
      case '\f': out += "\\f"; break;
      case '\n': out += "\\n"; break;
      case '\r': out += "\\r"; break;
      case '\t': out += "\\t"; break;
      default:
        if (static_cast<unsigned char>(c) < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", static_cast<unsigned>(c));
          out += buf;
        } else {
          out += c;
        }
    }
  }
  out += '"';
}

// Compact one-line object writer, keys in the order given.
class ObjectWriter {
 public:
  ObjectWriter& field(const std::string& k, const std::string& v) {
    key(k);
    append_quoted(out_, v);
    return *this;
  }
  ObjectWriter& field(const std::string& k, bool v) {
    key(k);
    out_ += v ? "true" : "false";
    return *this;
  }
  ObjectWriter& field(const std::string& k, const char* v) { return field(k, std::string(v)); }
  ObjectWriter& field(const std::string& k, int64_t v) {
    key(k);
    out_ += std::to_string(v);
    return *this;
  }
  ObjectWriter& field(const std::string& k, int v) { return field(k, static_cast<int64_t>(v)); }
  ObjectWriter& field(const std::string& k, double v) {
    key(k);
    out_ += number_text(v);
    return *this;
  }
  ObjectWriter& field(const std::string& k, float v) { return field(k, static_cast<double>(v)); }
  std::string str() const { return out_ + "}"; }

 private:
  void key(const std::string& k) {
    out_ += out_.size() > 1 ? "," : "";
    out_ += '"' + k + "\":";
  }
  std::string out_ = "{";
};

}  // namespace ctd::json
