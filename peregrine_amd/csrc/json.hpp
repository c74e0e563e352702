// Minimal JSON reader for checkpoint metadata: safetensors headers, the shard
// index (model.safetensors.index.json) and config.json. Host code only.
//
// Integers without a fraction or exponent are kept exactly (int64, or uint64
// above INT64_MAX), so byte offsets past 2^53 survive. Objects keep their
// insertion order; get() returns the last value of a repeated key. Nesting is
// limited to 64 levels so hostile input cannot exhaust the stack.
#pragma once

#include <stdint.h>
#include <stdlib.h>

#include <string>
#include <utility>
#include <vector>

namespace prg {
namespace json {

struct Value {
  enum Kind { kNull, kBool, kInt, kUint, kFloat, kString, kArray, kObject };
  Kind kind = kNull;
  bool b = false;
  int64_t i = 0;   // kInt
  uint64_t u = 0;  // kUint (> INT64_MAX)
  double f = 0.0;  // kFloat
  std::string s;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  const Value* get(const std::string& key) const {
    const Value* hit = nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) hit = &kv.second;
    return hit;
  }
  bool is_object() const { return kind == kObject; }
  bool is_array() const { return kind == kArray; }
  bool is_string() const { return kind == kString; }
  bool is_integer() const { return kind == kInt || kind == kUint; }
  bool is_number() const { return kind == kInt || kind == kUint || kind == kFloat; }
  // Non-negative integer as uint64 (false for negatives, floats, others).
  bool as_u64(uint64_t* out) const {
    if (kind == kUint) { *out = u; return true; }
    if (kind == kInt && i >= 0) { *out = static_cast<uint64_t>(i); return true; }
    return false;
  }
  double as_double() const {
    return kind == kFloat ? f : kind == kInt ? static_cast<double>(i) : kind == kUint ? static_cast<double>(u) : 0.0;
  }
};

class Parser {
 public:
  Parser(const char* p, size_t n) : p_(p), end_(p + n) {}

  bool parse(Value& out, std::string& err) {
    skip_ws();
    if (!value(out, 0)) {
      err = err_.empty() ? "malformed JSON" : err_;
      return false;
    }
    skip_ws();
    if (p_ != end_) {
      err = "trailing characters after JSON value";
      return false;
    }
    return true;
  }

 private:
  const char* p_;
  const char* end_;
  std::string err_;

  bool fail(const char* why) {
    if (err_.empty()) err_ = why;
    return false;
  }
  void skip_ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool literal(const char* word) {
    const char* q = p_;
    for (; *word; ++word, ++q)
      if (q >= end_ || *q != *word) return fail("invalid literal");
    p_ = q;
    return true;
  }

  bool value(Value& v, int depth) {
    if (depth > 64) return fail("JSON nested too deeply");
    if (p_ >= end_) return fail("unexpected end of JSON");
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = Value::kString; return string(v.s);
      case 't': v.kind = Value::kBool; v.b = true; return literal("true");
      case 'f': v.kind = Value::kBool; v.b = false; return literal("false");
      case 'n': v.kind = Value::kNull; return literal("null");
      default: return number(v);
    }
  }

  bool object(Value& v, int depth) {
    v.kind = Value::kObject;
    ++p_;
    skip_ws();
    if (p_ < end_ && *p_ == '}') { ++p_; return true; }
    for (;;) {
      skip_ws();
      if (p_ >= end_ || *p_ != '"') return fail("expected object key");
      std::string key;
      if (!string(key)) return false;
      skip_ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      ++p_;
      skip_ws();
      v.obj.emplace_back(std::move(key), Value{});
      if (!value(v.obj.back().second, depth + 1)) return false;
      skip_ws();
      if (p_ < end_ && *p_ == ',') { ++p_; continue; }
      if (p_ < end_ && *p_ == '}') { ++p_; return true; }
      return fail("expected ',' or '}'");
    }
  }

  bool array(Value& v, int depth) {
    v.kind = Value::kArray;
    ++p_;
    skip_ws();
    if (p_ < end_ && *p_ == ']') { ++p_; return true; }
    for (;;) {
      skip_ws();
      v.arr.emplace_back();
      if (!value(v.arr.back(), depth + 1)) return false;
      skip_ws();
      if (p_ < end_ && *p_ == ',') { ++p_; continue; }
      if (p_ < end_ && *p_ == ']') { ++p_; return true; }
      return fail("expected ',' or ']'");
    }
  }

  static int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }
  bool hex4(uint32_t* cp) {
    if (end_ - p_ < 4) return fail("truncated \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      const int h = hexval(p_[k]);
      if (h < 0) return fail("invalid \\u escape");
      v = v * 16 + static_cast<uint32_t>(h);
    }
    p_ += 4;
    *cp = v;
    return true;
  }
  static void put_utf8(std::string& s, uint32_t cp) {
    if (cp < 0x80) {
      s += static_cast<char>(cp);
    } else if (cp < 0x800) {
      s += static_cast<char>(0xC0 | (cp >> 6));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += static_cast<char>(0xE0 | (cp >> 12));
      s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    } else {
      s += static_cast<char>(0xF0 | (cp >> 18));
      s += static_cast<char>(0x80 | ((cp >> 12) & 0x3F));
      s += static_cast<char>(0x80 | ((cp >> 6) & 0x3F));
      s += static_cast<char>(0x80 | (cp & 0x3F));
    }
  }

  bool string(std::string& s) {
    ++p_;  // opening quote
    for (;;) {
      if (p_ >= end_) return fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if (static_cast<unsigned char>(c) < 0x20) return fail("control character in string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp = 0;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
            uint32_t lo = 0;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("unpaired surrogate");
            p_ += 2;
            if (!hex4(&lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("unpaired surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return fail("unpaired surrogate");
          }
          put_utf8(s, cp);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }

  bool number(Value& v) {
    const char* start = p_;
    bool neg = false;
    if (p_ < end_ && *p_ == '-') { neg = true; ++p_; }
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid value");
    if (*p_ == '0' && p_ + 1 < end_ && p_[1] >= '0' && p_[1] <= '9') return fail("leading zero");
    const char* digits = p_;
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    bool is_float = false;
    if (p_ < end_ && *p_ == '.') {
      is_float = true;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid fraction");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      is_float = true;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid exponent");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(start, p_);
    if (!is_float) {
      // exact integer: accumulate the magnitude with overflow checks
      uint64_t mag = 0;
      bool overflow = false;
      for (const char* q = digits; q < p_; ++q) {
        const uint64_t d = static_cast<uint64_t>(*q - '0');
        if (mag > (UINT64_MAX - d) / 10) { overflow = true; break; }
        mag = mag * 10 + d;
      }
      if (!overflow) {
        if (!neg) {
          if (mag <= static_cast<uint64_t>(INT64_MAX)) {
            v.kind = Value::kInt;
            v.i = static_cast<int64_t>(mag);
          } else {
            v.kind = Value::kUint;
            v.u = mag;
          }
          return true;
        }
        if (mag <= static_cast<uint64_t>(INT64_MAX) + 1) {
          v.kind = Value::kInt;
          v.i = mag == static_cast<uint64_t>(INT64_MAX) + 1 ? INT64_MIN : -static_cast<int64_t>(mag);
          return true;
        }
      }
    }
    v.kind = Value::kFloat;
    v.f = strtod(text.c_str(), nullptr);
    return true;
  }
};

inline bool parse(const char* p, size_t n, Value& out, std::string& err) {
  Parser ps(p, n);
  return ps.parse(out, err);
}

}  // namespace json
}  // namespace prg
