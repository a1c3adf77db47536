#include "json.h"

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "common.h"

namespace lcr {
namespace json {

Value Value::boolean(bool b) {
  Value v;
  v.kind_ = Kind::kBool;
  v.bool_ = b;
  return v;
}

Value Value::number(double d, bool integral) {
  Value v;
  v.kind_ = Kind::kNumber;
  v.number_ = d;
  v.integral_ = integral;
  v.int_ = integral ? static_cast<int64_t>(d) : 0;
  return v;
}

Value Value::integer(int64_t i) {
  Value v;
  v.kind_ = Kind::kNumber;
  v.number_ = static_cast<double>(i);
  v.integral_ = true;
  v.int_ = i;
  return v;
}

Value Value::string(std::string s) {
  Value v;
  v.kind_ = Kind::kString;
  v.string_ = std::move(s);
  return v;
}

Value Value::array() {
  Value v;
  v.kind_ = Kind::kArray;
  return v;
}

Value Value::object() {
  Value v;
  v.kind_ = Kind::kObject;
  return v;
}

bool Value::as_bool() const {
  LCR_CHECK(is_bool(), "JSON value is not a boolean");
  return bool_;
}

double Value::as_double() const {
  LCR_CHECK(is_number(), "JSON value is not a number");
  return integral_ ? static_cast<double>(int_) : number_;
}

int64_t Value::as_int64() const {
  LCR_CHECK(is_number(), "JSON value is not a number");
  return integral_ ? int_ : static_cast<int64_t>(number_);
}

int Value::as_int() const { return static_cast<int>(as_int64()); }

const std::string& Value::as_string() const {
  LCR_CHECK(is_string(), "JSON value is not a string");
  return string_;
}

const std::vector<Value>& Value::items() const {
  LCR_CHECK(is_array(), "JSON value is not an array");
  return array_;
}

void Value::push_back(Value v) {
  LCR_CHECK(is_array(), "JSON value is not an array");
  array_.push_back(std::move(v));
}

size_t Value::size() const {
  if (is_array()) return array_.size();
  if (is_object()) return object_.size();
  return 0;
}

bool Value::contains(const std::string& key) const {
  return is_object() && index_.count(key) != 0;
}

const Value* Value::find(const std::string& key) const {
  if (!is_object()) return nullptr;
  auto it = index_.find(key);
  return it == index_.end() ? nullptr : &object_[it->second].second;
}

const Value& Value::at(const std::string& key) const {
  const Value* v = find(key);
  LCR_CHECK(v != nullptr, "JSON object has no member \"" << key << "\"");
  return *v;
}

void Value::set(const std::string& key, Value v) {
  LCR_CHECK(is_object(), "JSON value is not an object");
  auto it = index_.find(key);
  if (it != index_.end()) {
    object_[it->second].second = std::move(v);
    return;
  }
  index_[key] = object_.size();
  object_.emplace_back(key, std::move(v));
}

const std::vector<std::pair<std::string, Value>>& Value::members() const {
  LCR_CHECK(is_object(), "JSON value is not an object");
  return object_;
}

namespace {

void dump_string(const std::string& s, std::string* out) {
  out->push_back('"');
  for (unsigned char c : s) {
    switch (c) {
      case '"': out->append("\\\""); break;
      case '\\': out->append("\\\\"); break;
      case '\n': out->append("\\n"); break;
      case '\r': out->append("\\r"); break;
      case '\t': out->append("\\t"); break;
      case '\b': out->append("\\b"); break;
      case '\f': out->append("\\f"); break;
      default:
        if (c < 0x20) {
          char buf[8];
          std::snprintf(buf, sizeof(buf), "\\u%04x", c);
          out->append(buf);
        } else {
          out->push_back(static_cast<char>(c));
        }
    }
  }
  out->push_back('"');
}

void dump_value(const Value& v, std::string* out) {
  switch (v.kind()) {
    case Value::Kind::kNull: out->append("null"); return;
    case Value::Kind::kBool: out->append(v.as_bool() ? "true" : "false"); return;
    case Value::Kind::kNumber: {
      char buf[40];
      if (v.is_integer()) {
        std::snprintf(buf, sizeof(buf), "%lld", static_cast<long long>(v.as_int64()));
      } else {
        std::snprintf(buf, sizeof(buf), "%.17g", v.as_double());
      }
      out->append(buf);
      return;
    }
    case Value::Kind::kString: dump_string(v.as_string(), out); return;
    case Value::Kind::kArray: {
      out->push_back('[');
      bool first = true;
      for (const Value& item : v.items()) {
        if (!first) out->push_back(',');
        first = false;
        dump_value(item, out);
      }
      out->push_back(']');
      return;
    }
    case Value::Kind::kObject: {
      out->push_back('{');
      bool first = true;
      for (const auto& member : v.members()) {
        if (!first) out->push_back(',');
        first = false;
        dump_string(member.first, out);
        out->push_back(':');
        dump_value(member.second, out);
      }
      out->push_back('}');
      return;
    }
  }
}

// Recursive-descent parser over a byte range.
class Parser {
 public:
  Parser(const char* begin, const char* end) : p_(begin), begin_(begin), end_(end) {}

  bool document(Value* out, std::string* error) {
    skip_ws();
    if (!value(out, 0)) {
      *error = error_;
      return false;
    }
    skip_ws();
    if (p_ != end_) {
      fail("trailing characters after the document");
      *error = error_;
      return false;
    }
    return true;
  }

 private:
  static constexpr int kMaxDepth = 512;

  bool fail(const char* what) {
    if (error_.empty()) {
      std::ostringstream oss;
      oss << what << " at byte " << (p_ - begin_);
      error_ = oss.str();
    }
    return false;
  }

  void skip_ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }

  bool literal(const char* word) {
    const size_t n = std::strlen(word);
    if (static_cast<size_t>(end_ - p_) < n || std::memcmp(p_, word, n) != 0) {
      return fail("invalid literal");
    }
    p_ += n;
    return true;
  }

  bool value(Value* out, int depth) {
    if (depth > kMaxDepth) return fail("nesting too deep");
    if (p_ >= end_) return fail("unexpected end of input");
    switch (*p_) {
      case '{': return object(out, depth);
      case '[': return array(out, depth);
      case '"': {
        std::string s;
        if (!string(&s)) return false;
        *out = Value::string(std::move(s));
        return true;
      }
      case 't':
        if (!literal("true")) return false;
        *out = Value::boolean(true);
        return true;
      case 'f':
        if (!literal("false")) return false;
        *out = Value::boolean(false);
        return true;
      case 'n':
        if (!literal("null")) return false;
        *out = Value::null();
        return true;
      default: return number(out);
    }
  }

  bool object(Value* out, int depth) {
    ++p_;  // '{'
    *out = Value::object();
    skip_ws();
    if (p_ < end_ && *p_ == '}') {
      ++p_;
      return true;
    }
    while (true) {
      skip_ws();
      if (p_ >= end_ || *p_ != '"') return fail("expected a member name");
      std::string key;
      if (!string(&key)) return false;
      skip_ws();
      if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
      ++p_;
      skip_ws();
      Value member;
      if (!value(&member, depth + 1)) return false;
      out->set(key, std::move(member));
      skip_ws();
      if (p_ >= end_) return fail("unterminated object");
      if (*p_ == ',') {
        ++p_;
        continue;
      }
      if (*p_ == '}') {
        ++p_;
        return true;
      }
      return fail("expected ',' or '}'");
    }
  }

  bool array(Value* out, int depth) {
    ++p_;  // '['
    *out = Value::array();
    skip_ws();
    if (p_ < end_ && *p_ == ']') {
      ++p_;
      return true;
    }
    while (true) {
      skip_ws();
      Value item;
      if (!value(&item, depth + 1)) return false;
      out->push_back(std::move(item));
      skip_ws();
      if (p_ >= end_) return fail("unterminated array");
      if (*p_ == ',') {
        ++p_;
        continue;
      }
      if (*p_ == ']') {
        ++p_;
        return true;
      }
      return fail("expected ',' or ']'");
    }
  }

  static int hex_digit(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  }

  bool hex4(uint32_t* out) {
    if (end_ - p_ < 4) return fail("truncated \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) {
      const int d = hex_digit(p_[i]);
      if (d < 0) return fail("invalid \\u escape");
      v = (v << 4) | static_cast<uint32_t>(d);
    }
    p_ += 4;
    *out = v;
    return true;
  }

  static void append_utf8(uint32_t cp, std::string* out) {
    if (cp < 0x80) {
      out->push_back(static_cast<char>(cp));
    } else if (cp < 0x800) {
      out->push_back(static_cast<char>(0xC0 | (cp >> 6)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
      out->push_back(static_cast<char>(0xE0 | (cp >> 12)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    } else {
      out->push_back(static_cast<char>(0xF0 | (cp >> 18)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 12) & 0x3F)));
      out->push_back(static_cast<char>(0x80 | ((cp >> 6) & 0x3F)));
      out->push_back(static_cast<char>(0x80 | (cp & 0x3F)));
    }
  }

  bool string(std::string* out) {
    ++p_;  // opening quote
    while (true) {
      if (p_ >= end_) return fail("unterminated string");
      const unsigned char c = static_cast<unsigned char>(*p_);
      if (c == '"') {
        ++p_;
        return true;
      }
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        out->push_back(static_cast<char>(c));
        ++p_;
        continue;
      }
      ++p_;
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': out->push_back('"'); break;
        case '\\': out->push_back('\\'); break;
        case '/': out->push_back('/'); break;
        case 'b': out->push_back('\b'); break;
        case 'f': out->push_back('\f'); break;
        case 'n': out->push_back('\n'); break;
        case 'r': out->push_back('\r'); break;
        case 't': out->push_back('\t'); break;
        case 'u': {
          uint32_t cp = 0;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp <= 0xDBFF) {
            // High surrogate: a low surrogate escape must follow.
            if (end_ - p_ < 6 || p_[0] != '\\' || p_[1] != 'u') {
              return fail("unpaired surrogate");
            }
            p_ += 2;
            uint32_t low = 0;
            if (!hex4(&low)) return false;
            if (low < 0xDC00 || low > 0xDFFF) return fail("invalid low surrogate");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (low - 0xDC00);
          } else if (cp >= 0xDC00 && cp <= 0xDFFF) {
            return fail("unpaired surrogate");
          }
          append_utf8(cp, out);
          break;
        }
        default: return fail("invalid escape");
      }
    }
  }

  bool number(Value* out) {
    const char* start = p_;
    bool integral = true;
    if (p_ < end_ && *p_ == '-') ++p_;
    if (p_ >= end_) return fail("invalid number");
    if (*p_ == '0') {
      ++p_;
    } else if (*p_ >= '1' && *p_ <= '9') {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    } else {
      return fail("invalid value");
    }
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid fraction");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      ++p_;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) ++p_;
      if (p_ >= end_ || *p_ < '0' || *p_ > '9') return fail("invalid exponent");
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') ++p_;
    }
    const std::string text(start, p_);
    if (integral) {
      errno = 0;
      char* stop = nullptr;
      const long long i = std::strtoll(text.c_str(), &stop, 10);
      if (errno == 0 && stop != nullptr && *stop == '\0') {
        *out = Value::integer(i);
        return true;
      }
    }
    *out = Value::number(std::strtod(text.c_str(), nullptr), false);
    return true;
  }

  const char* p_;
  const char* begin_;
  const char* end_;
  std::string error_;
};

}  // namespace

std::string Value::dump() const {
  std::string out;
  dump_value(*this, &out);
  return out;
}

bool parse(const char* begin, const char* end, Value* out, std::string* error) {
  Parser parser(begin, end);
  std::string local;
  return parser.document(out, error != nullptr ? error : &local);
}

bool parse(const std::string& text, Value* out, std::string* error) {
  return parse(text.data(), text.data() + text.size(), out, error);
}

}  // namespace json
}  // namespace lcr
