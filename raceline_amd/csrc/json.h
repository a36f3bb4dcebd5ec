// A small JSON reader for the header of .rlm model files (the reference parses it with
// NSJSONSerialization, src/model_file.mm:48-51). Objects keep their members in file order;
// numbers keep an exact 64-bit integer beside the double when they are written without a
// fraction or exponent (file offsets can pass 2^31). Host code only.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace rlq {
namespace json {

struct Value {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool b = false;
  double num = 0.0;
  int64_t i64 = 0;
  bool integral = false;                                   // written as an integer
  std::string str;
  std::vector<Value> arr;
  std::vector<std::pair<std::string, Value>> obj;

  const Value *get(const std::string &key) const {         // nullptr when absent or not an object
    if (kind != kObject) return nullptr;
    for (const auto &kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  bool is_number() const { return kind == kNumber; }
  bool is_string() const { return kind == kString; }
  bool is_object() const { return kind == kObject; }
  bool is_array() const { return kind == kArray; }
};

// Parses text[0, n). On a syntax error returns false with a message naming the offset.
class Parser {
 public:
  Parser(const char *text, size_t n) : p_(text), end_(text + n), begin_(text) {}

  bool parse(Value &out, std::string &err) {
    ws();
    if (!value(out, 0)) {
      err = err_;
      return false;
    }
    ws();
    if (p_ != end_) {
      err = at("trailing characters after the JSON value");
      return false;
    }
    return true;
  }

 private:
  const char *p_, *end_, *begin_;
  std::string err_;

  std::string at(const char *what) const { return std::string(what) + " at byte " + std::to_string(p_ - begin_); }
  bool fail(const char *what) {
    err_ = at(what);
    return false;
  }
  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char *s) {
    const char *q = p_;
    for (; *s; ++s, ++q)
      if (q >= end_ || *q != *s) return false;
    p_ = q;
    return true;
  }

  bool value(Value &v, int depth) {
    if (depth > 64) return fail("JSON nested too deeply");
    if (p_ >= end_) return fail("unexpected end of JSON");
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = Value::kString; return string(v.str);
      case 't': v.kind = Value::kBool; v.b = true; return lit("true") || fail("bad literal");
      case 'f': v.kind = Value::kBool; v.b = false; return lit("false") || fail("bad literal");
      case 'n': v.kind = Value::kNull; return lit("null") || fail("bad literal");
      default: return number(v);
    }
  }

  bool object(Value &v, int depth) {
    v.kind = Value::kObject;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == '}') {
      ++p_;
      return true;
    }
    for (;;) {
      ws();
      if (p_ >= end_ || *p_ != '"') return fail("expected a member name");
      std::string key;
      if (!string(key)) return false;
      ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      ++p_;
      ws();
      v.obj.emplace_back(std::move(key), Value());
      if (!value(v.obj.back().second, depth + 1)) return false;
      ws();
      if (p_ < end_ && *p_ == ',') {
        ++p_;
        continue;
      }
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      return fail("expected ',' or '}'");
    }
  }

  bool array(Value &v, int depth) {
    v.kind = Value::kArray;
    ++p_;
    ws();
    if (p_ < end_ && *p_ == ']') {
      ++p_;
      return true;
    }
    for (;;) {
      ws();
      v.arr.emplace_back();
      if (!value(v.arr.back(), depth + 1)) return false;
      ws();
      if (p_ < end_ && *p_ == ',') {
        ++p_;
        continue;
      }
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      return fail("expected ',' or ']'");
    }
  }

  static void utf8(std::string &s, uint32_t c) {
    if (c < 0x80) {
      s += (char)c;
    } else if (c < 0x800) {
      s += (char)(0xC0 | (c >> 6));
      s += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      s += (char)(0xE0 | (c >> 12));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    } else {
      s += (char)(0xF0 | (c >> 18));
      s += (char)(0x80 | ((c >> 12) & 0x3F));
      s += (char)(0x80 | ((c >> 6) & 0x3F));
      s += (char)(0x80 | (c & 0x3F));
    }
  }

  bool hex4(uint32_t &c) {
    if (end_ - p_ < 4) return fail("short \\u escape");
    c = 0;
    for (int i = 0; i < 4; ++i) {
      const char h = *p_++;
      c <<= 4;
      if (h >= '0' && h <= '9') c |= (uint32_t)(h - '0');
      else if (h >= 'a' && h <= 'f') c |= (uint32_t)(h - 'a' + 10);
      else if (h >= 'A' && h <= 'F') c |= (uint32_t)(h - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }

  bool string(std::string &out) {
    ++p_;   // the opening quote
    for (;;) {
      if (p_ >= end_) return fail("unterminated string");
      const char ch = *p_++;
      if (ch == '"') return true;
      if ((unsigned char)ch < 0x20) return fail("control character in a string");
      if (ch != '\\') {
        out += ch;
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
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
          uint32_t c;
          if (!hex4(c)) return false;
          if (c >= 0xD800 && c < 0xDC00) {   // a surrogate pair
            uint32_t lo;
            if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
            p_ += 2;
            if (!hex4(lo)) return false;
            if (lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(out, c);
          break;
        }
        default: return fail("bad escape");
      }
    }
  }

  bool number(Value &v) {
    const char *s = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("expected a value");
    while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad number");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("bad exponent");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(s, p_);
    v.kind = Value::kNumber;
    v.num = std::strtod(text.c_str(), nullptr);
    v.integral = integral && text.size() <= 19;
    if (v.integral) v.i64 = std::strtoll(text.c_str(), nullptr, 10);
    return true;
  }
};

}  // namespace json
}  // namespace rlq
