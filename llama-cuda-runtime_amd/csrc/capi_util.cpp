#include "capi_util.h"

#include "dtype.h"

namespace lcr {
namespace capi {
namespace {
thread_local std::string g_last_error;
}  // namespace

void set_error(const std::string& message) { g_last_error = message; }
void clear_error() { g_last_error.clear(); }

int hip_failure(const char* expr, hipError_t status) {
  std::ostringstream oss;
  oss << "HIP call failed: " << expr << ": " << hipGetErrorName(status) << ": "
      << hipGetErrorString(status);
  g_last_error = oss.str();
  return static_cast<int>(status);
}

}  // namespace capi
}  // namespace lcr

extern "C" const char* lcr_last_error_message(void) {
  return lcr::capi::g_last_error.c_str();
}

extern "C" const char* lcr_elem_name(void) { return lcr::kElemName; }
