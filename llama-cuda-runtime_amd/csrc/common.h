// Host-side error reporting, checkpoint element types and small helpers.
//
// Drop-in for the reference's src/common.h:12-54: the same lcr::Error type, the
// same LCR_CHECK / LCR_FAIL macros (file, line, condition text, message), the
// same DType enum and helper names, so host code and host tests written against
// the reference compile against this unchanged.
#pragma once

#include <cstddef>
#include <cstdint>
#include <sstream>
#include <stdexcept>
#include <string>

namespace lcr {

class Error : public std::runtime_error {
 public:
  explicit Error(const std::string& what) : std::runtime_error(what) {}
};

namespace detail {
[[noreturn]] void throw_failure(const char* file, int line, const char* cond,
                                const std::string& msg);
}  // namespace detail

// Release-mode checks. A failure throws lcr::Error whose text carries the file,
// the line, the condition and a formatted message:
//   LCR_CHECK(n > 0, "expected a positive length, got " << n);
#define LCR_CHECK(cond, msg)                                        \
  do {                                                              \
    if (!(cond)) {                                                  \
      std::ostringstream lcr_msg_stream_;                           \
      lcr_msg_stream_ << msg;                                       \
      ::lcr::detail::throw_failure(__FILE__, __LINE__, #cond,       \
                                   lcr_msg_stream_.str());          \
    }                                                               \
  } while (0)

#define LCR_FAIL(msg) LCR_CHECK(false, msg)

// Element types a safetensors checkpoint can hold. Only BF16, F16 and F32 are
// computed with; the others are described so the loader can name them.
enum class DType { kF32, kF16, kBF16, kI64, kI32, kI8, kU8, kBool };

size_t dtype_size(DType dt);
const char* dtype_name(DType dt);
DType dtype_from_string(const std::string& s);

// Next multiple of `alignment` (a power of two) at or above `value`.
inline size_t align_up(size_t value, size_t alignment) {
  return (value + alignment - 1) & ~(alignment - 1);
}

// "1.50 GiB"-style rendering for reports.
std::string format_bytes(size_t bytes);

}  // namespace lcr
