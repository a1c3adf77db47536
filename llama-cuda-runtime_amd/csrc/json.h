// A small self-contained JSON reader and writer.
//
// The reference parses config.json and safetensors headers with nlohmann/json,
// which its build downloads at configure time. This image has no network, so
// the runtime carries its own parser: enough of RFC 8259 for the documents a
// checkpoint directory holds (objects, arrays, strings with escapes including
// surrogate pairs, numbers, booleans, null). Object members keep their file
// order, which is what a safetensors header writer needs.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace lcr {
namespace json {

class Value {
 public:
  enum class Kind { kNull, kBool, kNumber, kString, kArray, kObject };

  Value() = default;
  static Value null() { return Value(); }
  static Value boolean(bool b);
  static Value number(double d, bool integral);
  static Value integer(int64_t i);
  static Value string(std::string s);
  static Value array();
  static Value object();

  Kind kind() const { return kind_; }
  bool is_null() const { return kind_ == Kind::kNull; }
  bool is_bool() const { return kind_ == Kind::kBool; }
  bool is_number() const { return kind_ == Kind::kNumber; }
  // A number written without a fraction or exponent that fits in int64.
  bool is_integer() const { return kind_ == Kind::kNumber && integral_; }
  bool is_string() const { return kind_ == Kind::kString; }
  bool is_array() const { return kind_ == Kind::kArray; }
  bool is_object() const { return kind_ == Kind::kObject; }

  bool as_bool() const;
  double as_double() const;
  int64_t as_int64() const;
  int as_int() const;
  float as_float() const { return static_cast<float>(as_double()); }
  const std::string& as_string() const;

  // Arrays.
  const std::vector<Value>& items() const;
  void push_back(Value v);
  size_t size() const;

  // Objects.
  bool contains(const std::string& key) const;
  const Value& at(const std::string& key) const;  // throws when absent
  const Value* find(const std::string& key) const;
  void set(const std::string& key, Value v);
  const std::vector<std::pair<std::string, Value>>& members() const;

  std::string dump() const;

 private:
  Kind kind_ = Kind::kNull;
  bool bool_ = false;
  bool integral_ = false;
  double number_ = 0.0;
  int64_t int_ = 0;
  std::string string_;
  std::vector<Value> array_;
  std::vector<std::pair<std::string, Value>> object_;
  std::map<std::string, size_t> index_;
};

// Parses a whole document. On malformed input returns false and fills `error`
// with the byte offset and reason; never throws for syntax errors.
bool parse(const char* begin, const char* end, Value* out, std::string* error);
bool parse(const std::string& text, Value* out, std::string* error);

}  // namespace json
}  // namespace lcr
