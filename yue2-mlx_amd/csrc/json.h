// Minimal JSON reader for the checkpoint manifest, config and safetensors
// header (host code). Objects keep their keys in a std::map; numbers keep
// both their text's integer-ness and a double value, which is what the
// reference's config checks distinguish (ar.cpp:160-191).
#pragma once
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace yuear {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  bool integer = false;  // a number written without fraction or exponent
  int64_t inum = 0;
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  bool is_object() const { return kind == Object; }
  bool is_array() const { return kind == Array; }
  bool is_string() const { return kind == String; }
  bool is_number() const { return kind == Number; }
  bool has(const std::string &k) const { return kind == Object && obj.count(k); }
  const Value *get(const std::string &k) const {
    if (kind != Object) return nullptr;
    auto it = obj.find(k);
    return it == obj.end() ? nullptr : &it->second;
  }
};

class Parser {
 public:
  explicit Parser(const std::string &text) : s_(text) {}
  Value parse() {
    Value v = value(0);
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string &s_;
  size_t i_ = 0;
  [[noreturn]] void fail(const char *what) {
    throw std::runtime_error(std::string("invalid JSON: ") + what + " at offset " +
                             std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r'))
      ++i_;
  }
  bool lit(const char *w) {
    size_t n = 0;
    while (w[n]) ++n;
    if (s_.compare(i_, n, w) == 0) {
      i_ += n;
      return true;
    }
    return false;
  }
  Value value(int depth) {
    if (depth > 64) fail("nesting too deep");
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    Value v;
    const char c = s_[i_];
    if (c == '{') {
      v.kind = Value::Object;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == '}') { ++i_; return v; }
      for (;;) {
        ws();
        if (i_ >= s_.size() || s_[i_] != '"') fail("expected a key");
        std::string k = string();
        ws();
        if (i_ >= s_.size() || s_[i_] != ':') fail("expected ':'");
        ++i_;
        v.obj[k] = value(depth + 1);
        ws();
        if (i_ < s_.size() && s_[i_] == ',') { ++i_; continue; }
        if (i_ < s_.size() && s_[i_] == '}') { ++i_; return v; }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind = Value::Array;
      ++i_;
      ws();
      if (i_ < s_.size() && s_[i_] == ']') { ++i_; return v; }
      for (;;) {
        v.arr.push_back(value(depth + 1));
        ws();
        if (i_ < s_.size() && s_[i_] == ',') { ++i_; continue; }
        if (i_ < s_.size() && s_[i_] == ']') { ++i_; return v; }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      v.str = string();
      return v;
    }
    if (lit("true")) { v.kind = Value::Bool; v.b = true; return v; }
    if (lit("false")) { v.kind = Value::Bool; v.b = false; return v; }
    if (lit("null")) return v;
    return number();
  }
  std::string string() {
    ++i_;  // opening quote
    std::string out;
    while (i_ < s_.size() && s_[i_] != '"') {
      char c = s_[i_++];
      if (c != '\\') { out += c; continue; }
      if (i_ >= s_.size()) fail("bad escape");
      c = s_[i_++];
      switch (c) {
      case '"': out += '"'; break;
      case '\\': out += '\\'; break;
      case '/': out += '/'; break;
      case 'b': out += '\b'; break;
      case 'f': out += '\f'; break;
      case 'n': out += '\n'; break;
      case 'r': out += '\r'; break;
      case 't': out += '\t'; break;
      case 'u': {
        if (i_ + 4 > s_.size()) fail("bad \\u escape");
        const unsigned cp = unsigned(std::strtoul(s_.substr(i_, 4).c_str(), nullptr, 16));
        i_ += 4;
        if (cp < 0x80) {
          out += char(cp);
        } else if (cp < 0x800) {
          out += char(0xC0 | (cp >> 6));
          out += char(0x80 | (cp & 0x3F));
        } else {
          out += char(0xE0 | (cp >> 12));
          out += char(0x80 | ((cp >> 6) & 0x3F));
          out += char(0x80 | (cp & 0x3F));
        }
        break;
      }
      default: fail("bad escape");
      }
    }
    if (i_ >= s_.size()) fail("unterminated string");
    ++i_;
    return out;
  }
  Value number() {
    const size_t start = i_;
    bool integer = true;
    if (i_ < s_.size() && s_[i_] == '-') ++i_;
    while (i_ < s_.size()) {
      const char c = s_[i_];
      if (c >= '0' && c <= '9') { ++i_; continue; }
      if (c == '.' || c == 'e' || c == 'E' || c == '+' || c == '-') { integer = false; ++i_; continue; }
      break;
    }
    if (i_ == start) fail("unexpected character");
    const std::string t = s_.substr(start, i_ - start);
    char *end = nullptr;
    Value v;
    v.kind = Value::Number;
    v.num = std::strtod(t.c_str(), &end);
    if (!end || *end) fail("bad number");
    v.integer = integer;
    if (integer) v.inum = std::strtoll(t.c_str(), nullptr, 10);
    return v;
  }
};

inline Value parse(const std::string &text) { return Parser(text).parse(); }

}  // namespace json
}  // namespace yuear
