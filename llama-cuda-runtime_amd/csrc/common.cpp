#include "common.h"

#include <cstdio>

namespace lcr {

namespace detail {

void fail_check(const CheckSite& site, const std::string& message) {
  std::string text = message.empty() ? std::string("check failed") : message;
  text += " [check `";
  text += site.condition;
  text += "` at ";
  text += site.file;
  text += ":";
  text += std::to_string(site.line);
  text += "]";
  throw Error(text);
}

}  // namespace detail

namespace {

struct ElementType {
  DType type;
  const char* header_name;  // spelling in a safetensors header
  uint8_t bytes;
};

// One row per DType, in enum order.
constexpr ElementType kElementTypes[] = {
    {DType::kF32, "F32", 4}, {DType::kF16, "F16", 2}, {DType::kBF16, "BF16", 2},
    {DType::kI64, "I64", 8}, {DType::kI32, "I32", 4}, {DType::kI8, "I8", 1},
    {DType::kU8, "U8", 1},   {DType::kBool, "BOOL", 1},
};

const ElementType& element_type(DType dt) {
  for (const ElementType& e : kElementTypes) {
    if (e.type == dt) return e;
  }
  LCR_FAIL("DType value " << static_cast<int>(dt) << " has no table entry");
}

}  // namespace

size_t dtype_size(DType dt) { return element_type(dt).bytes; }

const char* dtype_name(DType dt) { return element_type(dt).header_name; }

DType dtype_from_string(const std::string& s) {
  for (const ElementType& e : kElementTypes) {
    if (s == e.header_name) return e.type;
  }
  // Float64 is a valid safetensors type, just not one this runtime computes in.
  LCR_CHECK(s != "F64", "F64 tensors are not supported");
  LCR_FAIL("unknown safetensors dtype \"" << s << "\"");
}

std::string format_bytes(size_t bytes) {
  if (bytes < 1024) return std::to_string(bytes) + " B";
  const char* const units[] = {"KiB", "MiB", "GiB", "TiB", "PiB"};
  int unit = 0;
  size_t scale = 1024;
  while (unit + 1 < 5 && bytes / scale >= 1024) {
    scale *= 1024;
    ++unit;
  }
  char text[40];
  std::snprintf(text, sizeof(text), "%.2f %s",
                static_cast<double>(bytes) / static_cast<double>(scale), units[unit]);
  return text;
}

}  // namespace lcr
