#include "json.hpp"

#include <cmath>
#include <cstdlib>
#include <fstream>
#include <sstream>

namespace fiber::json {

bool Value::as_bool() const {
  if (kind_ != Bool) throw Error("json: not a boolean");
  return b_;
}
double Value::as_number() const {
  if (kind_ != Number) throw Error("json: not a number");
  return num_;
}
int64_t Value::as_int() const {
  const double v = as_number();
  if (v != std::floor(v) || std::fabs(v) > 9.007199254740992e15) throw Error("json: " + str_ + " is not an integer");
  return (int64_t)v;
}
const std::string& Value::as_string() const {
  if (kind_ != String) throw Error("json: not a string");
  return str_;
}
const std::vector<Value>& Value::items() const {
  if (kind_ != Array) throw Error("json: not an array");
  return arr_;
}
const std::vector<std::pair<std::string, Value>>& Value::members() const {
  if (kind_ != Object) throw Error("json: not an object");
  return obj_;
}
const Value* Value::find(const std::string& key) const {
  if (kind_ != Object) return nullptr;
  for (const auto& kv : obj_)
    if (kv.first == key) return &kv.second;
  return nullptr;
}
const Value& Value::at(const std::string& key) const {
  const Value* v = find(key);
  if (!v) throw Error("json: missing key \"" + key + "\"");
  return *v;
}
std::string Value::get_string(const std::string& key, const std::string& def) const {
  const Value* v = find(key);
  return v && !v->is_null() ? v->as_string() : def;
}
int64_t Value::get_int(const std::string& key, int64_t def) const {
  const Value* v = find(key);
  return v && !v->is_null() ? v->as_int() : def;
}
double Value::get_number(const std::string& key, double def) const {
  const Value* v = find(key);
  return v && !v->is_null() ? v->as_number() : def;
}
bool Value::get_bool(const std::string& key, bool def) const {
  const Value* v = find(key);
  return v && !v->is_null() ? v->as_bool() : def;
}

class Parser {
 public:
  explicit Parser(const std::string& s) : s_(s) {}

  Value document() {
    Value v = value(0);
    ws();
    if (i_ != s_.size()) fail("trailing characters");
    return v;
  }

 private:
  const std::string& s_;
  size_t i_ = 0;

  [[noreturn]] void fail(const std::string& what) const {
    throw Error("json: " + what + " at byte " + std::to_string(i_));
  }
  void ws() {
    while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) i_++;
  }
  bool lit(const char* w) {
    size_t n = 0;
    while (w[n]) n++;
    if (s_.compare(i_, n, w) != 0) return false;
    i_ += n;
    return true;
  }

  Value value(int depth) {
    if (depth > 512) fail("nesting too deep");
    ws();
    if (i_ >= s_.size()) fail("unexpected end");
    Value v;
    const char c = s_[i_];
    if (c == '{') {
      v.kind_ = Value::Object;
      i_++;
      ws();
      if (i_ < s_.size() && s_[i_] == '}') {
        i_++;
        return v;
      }
      for (;;) {
        ws();
        if (i_ >= s_.size() || s_[i_] != '"') fail("expected a key");
        std::string k = string();
        ws();
        if (i_ >= s_.size() || s_[i_] != ':') fail("expected ':'");
        i_++;
        v.obj_.emplace_back(std::move(k), value(depth + 1));
        ws();
        if (i_ < s_.size() && s_[i_] == ',') {
          i_++;
          continue;
        }
        if (i_ < s_.size() && s_[i_] == '}') {
          i_++;
          return v;
        }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      v.kind_ = Value::Array;
      i_++;
      ws();
      if (i_ < s_.size() && s_[i_] == ']') {
        i_++;
        return v;
      }
      for (;;) {
        v.arr_.push_back(value(depth + 1));
        ws();
        if (i_ < s_.size() && s_[i_] == ',') {
          i_++;
          continue;
        }
        if (i_ < s_.size() && s_[i_] == ']') {
          i_++;
          return v;
        }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      v.kind_ = Value::String;
      v.str_ = string();
      return v;
    }
    if (lit("true")) {
      v.kind_ = Value::Bool;
      v.b_ = true;
      return v;
    }
    if (lit("false")) {
      v.kind_ = Value::Bool;
      return v;
    }
    if (lit("null")) return v;
    if (c == '-' || (c >= '0' && c <= '9')) {
      const size_t b = i_;
      if (s_[i_] == '-') i_++;
      while (i_ < s_.size() && ((s_[i_] >= '0' && s_[i_] <= '9') || s_[i_] == '.' || s_[i_] == 'e' || s_[i_] == 'E' ||
                                s_[i_] == '+' || s_[i_] == '-'))
        i_++;
      v.kind_ = Value::Number;
      v.str_ = s_.substr(b, i_ - b);
      char* end = nullptr;
      v.num_ = std::strtod(v.str_.c_str(), &end);
      if (end != v.str_.c_str() + v.str_.size()) fail("bad number " + v.str_);
      return v;
    }
    fail(std::string("unexpected character '") + c + "'");
  }

  static void put_utf8(std::string& out, uint32_t cp) {
    if (cp < 0x80) {
      out += (char)cp;
    } else if (cp < 0x800) {
      out += (char)(0xC0 | (cp >> 6));
      out += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      out += (char)(0xE0 | (cp >> 12));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    } else {
      out += (char)(0xF0 | (cp >> 18));
      out += (char)(0x80 | ((cp >> 12) & 0x3F));
      out += (char)(0x80 | ((cp >> 6) & 0x3F));
      out += (char)(0x80 | (cp & 0x3F));
    }
  }

  uint32_t hex4() {
    if (i_ + 4 > s_.size()) fail("short \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; k++) {
      const char h = s_[i_++];
      v <<= 4;
      if (h >= '0' && h <= '9') v |= h - '0';
      else if (h >= 'a' && h <= 'f') v |= h - 'a' + 10;
      else if (h >= 'A' && h <= 'F') v |= h - 'A' + 10;
      else fail("bad \\u escape");
    }
    return v;
  }

  std::string string() {
    i_++;  // opening quote
    std::string out;
    for (;;) {
      if (i_ >= s_.size()) fail("unterminated string");
      const char c = s_[i_++];
      if (c == '"') return out;
      if ((unsigned char)c < 0x20) fail("control character in string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i_ >= s_.size()) fail("unterminated escape");
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
          if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one must follow
            if (i_ + 6 <= s_.size() && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
              i_ += 2;
              const uint32_t lo = hex4();
              if (lo >= 0xDC00 && lo < 0xE000) cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
              else fail("unpaired surrogate");
            } else {
              fail("unpaired surrogate");
            }
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            fail("unpaired surrogate");
          }
          put_utf8(out, cp);
          break;
        }
        default: fail(std::string("bad escape \\") + e);
      }
    }
  }
};

Value parse(const std::string& text) { return Parser(text).document(); }

Value parse_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw Error("json: cannot open " + path);
  std::ostringstream ss;
  ss << f.rdbuf();
  try {
    return parse(ss.str());
  } catch (const Error& e) {
    throw Error(std::string(e.what()) + " in " + path);
  }
}

}  // namespace fiber::json
