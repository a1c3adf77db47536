// Host-side error type, release-mode checks and checkpoint element types.
//
// The names are the reference's host interface (src/common.h:12-54: lcr::Error,
// LCR_CHECK / LCR_FAIL, DType with dtype_size / dtype_name /
// dtype_from_string, align_up, format_bytes), so host code and host tests
// written against it compile here unchanged. The implementation is this
// build's own: a failing check hands its site and streamed message to one
// out-of-line function, and every element-type query reads one table.
#pragma once

#include <cstddef>
#include <cstdint>
#include <sstream>
#include <stdexcept>
#include <string>

namespace lcr {

class Error : public std::runtime_error {
 public:
  using std::runtime_error::runtime_error;
};

namespace detail {

// Source location and condition text of a check.
struct CheckSite {
  const char* file;
  int line;
  const char* condition;
};

// Accumulates the `<<`-streamed message of a failing check.
class CheckMessage {
 public:
  template <typename T>
  CheckMessage& operator<<(const T& value) {
    text_ << value;
    return *this;
  }
  std::string str() const { return text_.str(); }

 private:
  std::ostringstream text_;
};

// Throws lcr::Error: "<message> [check `<condition>` at <file>:<line>]".
[[noreturn]] void fail_check(const CheckSite& site, const std::string& message);

}  // namespace detail

// Stays in release builds. The message is only formatted on failure:
//   LCR_CHECK(n > 0, "expected a positive length, got " << n);
#define LCR_CHECK(cond, msg)                                                        \
  do {                                                                              \
    if (!(cond)) {                                                                  \
      ::lcr::detail::fail_check(::lcr::detail::CheckSite{__FILE__, __LINE__, #cond}, \
                                (::lcr::detail::CheckMessage() << msg).str());      \
    }                                                                               \
  } while (0)

#define LCR_FAIL(msg) LCR_CHECK(false, msg)

// Element types a safetensors checkpoint may hold. The token loop computes in
// BF16 or F16 (one per build) and F32; the integer types are named so that the
// loader can describe a checkpoint that carries them.
enum class DType { kF32, kF16, kBF16, kI64, kI32, kI8, kU8, kBool };

size_t dtype_size(DType dt);
const char* dtype_name(DType dt);
// Parses the safetensors header spelling ("BF16", "F32", ...).
DType dtype_from_string(const std::string& s);

// Smallest multiple of `alignment` (a power of two) that is >= value.
inline size_t align_up(size_t value, size_t alignment) {
  return (value + alignment - 1) & ~(alignment - 1);
}

// Binary-prefixed size for reports: "812 B", "4.00 KiB", "2.30 GiB".
std::string format_bytes(size_t bytes);

}  // namespace lcr
