// json_min.hpp — a small JSON reader for safetensors headers, weight-map
// indexes and model config files (objects, arrays, strings with escapes,
// numbers, booleans, null). Parse errors throw std::runtime_error.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace kiln {
namespace json {

struct Value {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  bool is_object() const { return kind == Object; }
  bool is_array() const { return kind == Array; }
  bool is_string() const { return kind == String; }
  bool is_number() const { return kind == Number; }
  const Value* get(const std::string& key) const {
    if (kind != Object) return nullptr;
    auto it = obj.find(key);
    return it == obj.end() ? nullptr : &it->second;
  }
};

class Parser {
 public:
  explicit Parser(const std::string& text) : s_(text) {}

  Value parse() {
    Value v = value();
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;

  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("json: ") + what + " at offset " + std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\n' || s_[i_] == '\r' || s_[i_] == '\t')) ++i_;
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
  bool literal(const char* lit) {
    size_t n = 0;
    while (lit[n]) ++n;
    if (s_.compare(i_, n, lit) == 0) {
      i_ += n;
      return true;
    }
    return false;
  }

  Value value() {
    const char c = peek();
    Value v;
    if (c == '{') {
      v.kind = Value::Object;
      ++i_;
      if (peek() == '}') {
        ++i_;
        return v;
      }
      for (;;) {
        if (peek() != '"') fail("expected key");
        std::string key = string();
        expect(':');
        v.obj[key] = value();
        const char d = peek();
        ++i_;
        if (d == '}') break;
        if (d != ',') fail("expected , or }");
      }
    } else if (c == '[') {
      v.kind = Value::Array;
      ++i_;
      if (peek() == ']') {
        ++i_;
        return v;
      }
      for (;;) {
        v.arr.push_back(value());
        const char d = peek();
        ++i_;
        if (d == ']') break;
        if (d != ',') fail("expected , or ]");
      }
    } else if (c == '"') {
      v.kind = Value::String;
      v.str = string();
    } else if (literal("true")) {
      v.kind = Value::Bool;
      v.b = true;
    } else if (literal("false")) {
      v.kind = Value::Bool;
    } else if (literal("null")) {
      v.kind = Value::Null;
    } else {
      v.kind = Value::Number;
      const char* start = s_.c_str() + i_;
      char* end = nullptr;
      v.num = std::strtod(start, &end);
      if (end == start) fail("bad value");
      i_ += (size_t)(end - start);
    }
    return v;
  }

  static void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xc0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      out += (char)(0xe0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3f));
      out += (char)(0x80 | (cp & 0x3f));
    } else {
      out += (char)(0xf0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3f));
      out += (char)(0x80 | ((cp >> 6) & 0x3f));
      out += (char)(0x80 | (cp & 0x3f));
    }
  }

  uint32_t hex4() {
    if (i_ + 4 > s_.size()) fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const char h = s_[i_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= (uint32_t)(h - '0');
      else if (h >= 'a' && h <= 'f') v |= (uint32_t)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') v |= (uint32_t)(h - 'A' + 10);
      else fail("bad \\u escape");
    }
    return v;
  }

  std::string string() {
    expect('"');
    std::string out;
    while (i_ < s_.size()) {
      const char c = s_[i_++];
      if (c == '"') return out;
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) break;
      const char e = s_[i_++];
      switch (e) {
        case '"': out += '"'; break;
        case '\\': out += '\\'; break;
        case '/': out += '/'; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u': {
          uint32_t cp = hex4();
          if (cp >= 0xd800 && cp < 0xdc00 && i_ + 6 <= s_.size() && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
            i_ += 2;
            const uint32_t lo = hex4();
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          put_utf8(out, cp);
          break;
        }
        default: fail("bad escape");
      }
    }
    fail("unterminated string");
  }
};

inline Value parse(const std::string& text) { return Parser(text).parse(); }

}  // namespace json
}  // namespace kiln
