// Minimal JSON reader for the model directory's files (config.json,
// tokenizer.json, safetensors headers, sentence-transformers configs).
// RFC 8259 values; strings are decoded to UTF-8 (\uXXXX escapes, surrogate
// pairs included); numbers are kept as double and as their source text.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

namespace fiber::json {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

class Value {
 public:
  enum Kind { Null, Bool, Number, String, Array, Object };

  Kind kind() const { return kind_; }
  bool is_null() const { return kind_ == Null; }
  bool is_object() const { return kind_ == Object; }
  bool is_array() const { return kind_ == Array; }
  bool is_string() const { return kind_ == String; }
  bool is_number() const { return kind_ == Number; }

  bool as_bool() const;
  double as_number() const;
  int64_t as_int() const;  // throws unless the number is integral
  const std::string& as_string() const;
  const std::vector<Value>& items() const;                         // array elements
  const std::vector<std::pair<std::string, Value>>& members() const;  // object members, in file order

  // Object member by key (first occurrence), or nullptr.
  const Value* find(const std::string& key) const;
  // Object member by key; throws when absent.
  const Value& at(const std::string& key) const;
  // Member value or a default when absent or null.
  std::string get_string(const std::string& key, const std::string& def = "") const;
  int64_t get_int(const std::string& key, int64_t def = 0) const;
  double get_number(const std::string& key, double def = 0) const;
  bool get_bool(const std::string& key, bool def = false) const;

 private:
  friend class Parser;
  Kind kind_ = Null;
  bool b_ = false;
  double num_ = 0;
  std::string str_;  // String value, or a Number's source text
  std::vector<Value> arr_;
  std::vector<std::pair<std::string, Value>> obj_;
};

Value parse(const std::string& text);
Value parse_file(const std::string& path);

}  // namespace fiber::json
