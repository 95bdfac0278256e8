// A small JSON reader for the checkpoint's config files and the safetensors header.
// It accepts the JSON grammar (objects, arrays, strings with escapes, numbers, true, false,
// null) and rejects anything else with a message that names the byte offset.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace s1 {

struct JsonValue {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0.0;
  bool is_int = false;   // the literal had no fraction or exponent
  int64_t i = 0;         // valid when is_int
  std::string str;
  std::vector<JsonValue> arr;
  std::vector<std::pair<std::string, JsonValue>> obj;  // keeps file order

  const JsonValue* get(const std::string& key) const {
    if (kind != Object) return nullptr;
    for (const auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  const JsonValue* path(std::initializer_list<const char*> keys) const {
    const JsonValue* v = this;
    for (const char* k : keys) {
      if (!v) return nullptr;
      v = v->get(k);
    }
    return v;
  }
};

class JsonParser {
 public:
  JsonParser(const char* s, size_t n) : s_(s), n_(n) {}

  JsonValue parse() {
    JsonValue v = value();
    ws();
    if (p_ != n_) fail("trailing characters");
    return v;
  }

 private:
  const char* s_;
  size_t n_;
  size_t p_ = 0;
  int depth_ = 0;

  [[noreturn]] void fail(const char* what) const {
    throw std::runtime_error(std::string("json: ") + what + " at byte " + std::to_string(p_));
  }
  void ws() {
    while (p_ < n_ && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\n' || s_[p_] == '\r')) ++p_;
  }
  bool lit(const char* w) {
    size_t k = 0;
    while (w[k]) {
      if (p_ + k >= n_ || s_[p_ + k] != w[k]) return false;
      ++k;
    }
    p_ += k;
    return true;
  }
  JsonValue value() {
    ws();
    if (p_ >= n_) fail("unexpected end");
    if (++depth_ > 256) fail("nesting too deep");
    JsonValue v;
    char c = s_[p_];
    if (c == '{') {
      v.kind = JsonValue::Object;
      ++p_;
      ws();
      if (p_ < n_ && s_[p_] == '}') {
        ++p_;
      } else {
        for (;;) {
          ws();
          if (p_ >= n_ || s_[p_] != '"') fail("expected a key");
          std::string k = string();
          ws();
          if (p_ >= n_ || s_[p_] != ':') fail("expected ':'");
          ++p_;
          JsonValue item = value();
          v.obj.emplace_back(std::move(k), std::move(item));
          ws();
          if (p_ < n_ && s_[p_] == ',') { ++p_; continue; }
          if (p_ < n_ && s_[p_] == '}') { ++p_; break; }
          fail("expected ',' or '}'");
        }
      }
    } else if (c == '[') {
      v.kind = JsonValue::Array;
      ++p_;
      ws();
      if (p_ < n_ && s_[p_] == ']') {
        ++p_;
      } else {
        for (;;) {
          v.arr.push_back(value());
          ws();
          if (p_ < n_ && s_[p_] == ',') { ++p_; continue; }
          if (p_ < n_ && s_[p_] == ']') { ++p_; break; }
          fail("expected ',' or ']'");
        }
      }
    } else if (c == '"') {
      v.kind = JsonValue::String;
      v.str = string();
    } else if (lit("true")) {
      v.kind = JsonValue::Bool;
      v.b = true;
    } else if (lit("false")) {
      v.kind = JsonValue::Bool;
    } else if (lit("null")) {
      v.kind = JsonValue::Null;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      v.kind = JsonValue::Number;
      size_t st = p_;
      bool frac = false;
      if (s_[p_] == '-') ++p_;
      while (p_ < n_ && ((s_[p_] >= '0' && s_[p_] <= '9') || s_[p_] == '.' || s_[p_] == 'e' ||
                         s_[p_] == 'E' || s_[p_] == '+' || s_[p_] == '-')) {
        if (s_[p_] == '.' || s_[p_] == 'e' || s_[p_] == 'E') frac = true;
        ++p_;
      }
      std::string t(s_ + st, p_ - st);
      char* end = nullptr;
      v.num = std::strtod(t.c_str(), &end);
      if (end == t.c_str() || *end != 0) fail("bad number");
      if (!frac) {
        v.is_int = true;
        v.i = std::strtoll(t.c_str(), nullptr, 10);
      }
    } else {
      fail("unexpected character");
    }
    --depth_;
    return v;
  }
  std::string string() {
    ++p_;  // opening quote
    std::string out;
    while (p_ < n_ && s_[p_] != '"') {
      char c = s_[p_++];
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (p_ >= n_) fail("bad escape");
      char e = s_[p_++];
      switch (e) {
        case '"': out.push_back('"'); break;
        case '\\': out.push_back('\\'); break;
        case '/': out.push_back('/'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'n': out.push_back('\n'); break;
        case 'r': out.push_back('\r'); break;
        case 't': out.push_back('\t'); break;
        case 'u': {
          if (p_ + 4 > n_) fail("bad \\u escape");
          unsigned cp = std::strtoul(std::string(s_ + p_, 4).c_str(), nullptr, 16);
          p_ += 4;
          // Names in these files are ASCII; other code points are kept as UTF-8.
          if (cp < 0x80) {
            out.push_back(char(cp));
          } else if (cp < 0x800) {
            out.push_back(char(0xC0 | (cp >> 6)));
            out.push_back(char(0x80 | (cp & 0x3F)));
          } else {
            out.push_back(char(0xE0 | (cp >> 12)));
            out.push_back(char(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back(char(0x80 | (cp & 0x3F)));
          }
          break;
        }
        default: fail("bad escape");
      }
    }
    if (p_ >= n_) fail("unterminated string");
    ++p_;
    return out;
  }
};

inline JsonValue parse_json(const std::string& text) {
  JsonParser p(text.data(), text.size());
  return p.parse();
}

}  // namespace s1
