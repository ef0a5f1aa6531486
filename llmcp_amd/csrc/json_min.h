// json_min.h -- minimal JSON reader for the embedded weight manifest.
//
// The reference parses the manifest with llvm::json (WeightArena.cpp:54-60);
// this build has no LLVM development libraries, so the loader uses this small
// recursive-descent parser.  It accepts RFC 8259 JSON and keeps integers
// exact (int64) when they have no fraction or exponent.
#pragma once

#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace llmcp_q8 {
namespace json {

struct Value {
  enum Kind { Null, Bool, Int, Double, String, Array, Object } kind = Null;
  bool b = false;
  int64_t i = 0;
  double d = 0.0;
  std::string s;
  std::vector<Value> arr;
  std::map<std::string, Value> obj;

  const Value *get(const std::string &key) const {
    if (kind != Object) return nullptr;
    auto it = obj.find(key);
    return it == obj.end() ? nullptr : &it->second;
  }
  bool is_int() const { return kind == Int; }
  bool is_string() const { return kind == String; }
};

class Parser {
 public:
  Parser(const char *p, size_t n) : p_(p), end_(p + n) {}

  bool parse(Value &out) {
    skip();
    if (!value(out, 0)) return false;
    skip();
    return p_ == end_;
  }

 private:
  const char *p_;
  const char *end_;

  void skip() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t'))
      ++p_;
  }

  bool lit(const char *w) {
    const char *q = p_;
    for (; *w; ++w, ++q)
      if (q >= end_ || *q != *w) return false;
    p_ = q;
    return true;
  }

  static int hex(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }

  static void utf8(std::string &s, uint32_t cp) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xc0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
      s += (char)(0xe0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3f));
      s += (char)(0x80 | (cp & 0x3f));
    } else {
      s += (char)(0xf0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3f));
      s += (char)(0x80 | ((cp >> 6) & 0x3f));
      s += (char)(0x80 | (cp & 0x3f));
    }
  }

  bool u4(uint32_t &cp) {
    if (end_ - p_ < 4) return false;
    cp = 0;
    for (int k = 0; k < 4; ++k) {
      int h = hex(p_[k]);
      if (h < 0) return false;
      cp = cp * 16 + (uint32_t)h;
    }
    p_ += 4;
    return true;
  }

  bool string(std::string &s) {
    if (p_ >= end_ || *p_ != '"') return false;
    ++p_;
    while (p_ < end_ && *p_ != '"') {
      unsigned char c = (unsigned char)*p_;
      if (c < 0x20) return false;
      if (c != '\\') {
        s += (char)c;
        ++p_;
        continue;
      }
      if (++p_ >= end_) return false;
      char e = *p_++;
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
          uint32_t cp;
          if (!u4(cp)) return false;
          if (cp >= 0xd800 && cp < 0xdc00) {
            uint32_t lo;
            if (!lit("\\u") || !u4(lo) || lo < 0xdc00 || lo >= 0xe000)
              return false;
            cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
          }
          utf8(s, cp);
          break;
        }
        default: return false;
      }
    }
    if (p_ >= end_) return false;
    ++p_;
    return true;
  }

  bool number(Value &v) {
    const char *start = p_;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
    if (*p_ == '0') {
      ++p_;
    } else {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    std::string text(start, p_);
    if (integral) {
      errno = 0;
      char *stop = nullptr;
      long long x = std::strtoll(text.c_str(), &stop, 10);
      if (errno == 0 && stop && *stop == '\0') {
        v.kind = Value::Int;
        v.i = x;
        v.d = (double)x;
        return true;
      }
    }
    v.kind = Value::Double;
    v.d = std::strtod(text.c_str(), nullptr);
    return true;
  }

  bool value(Value &v, int depth) {
    if (depth > 64 || p_ >= end_) return false;
    char c = *p_;
    if (c == '{') {
      ++p_;
      v.kind = Value::Object;
      skip();
      if (p_ < end_ && *p_ == '}') {
        ++p_;
        return true;
      }
      while (true) {
        skip();
        std::string key;
        if (!string(key)) return false;
        skip();
        if (p_ >= end_ || *p_ != ':') return false;
        ++p_;
        skip();
        Value item;
        if (!value(item, depth + 1)) return false;
        v.obj[key] = std::move(item);
        skip();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = Value::Array;
      skip();
      if (p_ < end_ && *p_ == ']') {
        ++p_;
        return true;
      }
      while (true) {
        skip();
        Value item;
        if (!value(item, depth + 1)) return false;
        v.arr.push_back(std::move(item));
        skip();
        if (p_ < end_ && *p_ == ',') {
          ++p_;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          ++p_;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v.kind = Value::String;
      return string(v.s);
    }
    if (lit("true")) {
      v.kind = Value::Bool;
      v.b = true;
      return true;
    }
    if (lit("false")) {
      v.kind = Value::Bool;
      return true;
    }
    if (lit("null")) return true;
    return number(v);
  }
};

}  // namespace json
}  // namespace llmcp_q8
