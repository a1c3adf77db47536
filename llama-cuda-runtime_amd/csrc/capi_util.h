// Error plumbing for the extern "C" entry points: argument checks record the
// reference's message text in a thread-local string and return
// LCR_ERR_ARGUMENT; HIP failures return the hipError_t. Nothing throws across
// the C boundary.
#pragma once

#include <hip/hip_runtime.h>

#include <sstream>
#include <string>

#include "../../include/lcr_kernels.h"
#include "hip_utils.h"

namespace lcr {
namespace capi {

void set_error(const std::string& message);
void clear_error();
int hip_failure(const char* expr, hipError_t status);
// Runs `body`, mapping an lcr::Error or std::exception to LCR_ERR_ARGUMENT.
template <typename F>
int guarded(F&& body) {
  try {
    return body();
  } catch (const std::exception& e) {
    set_error(e.what());
    return LCR_ERR_ARGUMENT;
  }
}

}  // namespace capi
}  // namespace lcr

#define CAPI_CHECK(cond, msg)                       \
  do {                                              \
    if (!(cond)) {                                  \
      std::ostringstream capi_msg_;                 \
      capi_msg_ << msg;                             \
      ::lcr::capi::set_error(capi_msg_.str());      \
      return LCR_ERR_ARGUMENT;                      \
    }                                               \
  } while (0)

#define CAPI_HIP(expr)                                          \
  do {                                                          \
    const hipError_t capi_status_ = (expr);                     \
    if (capi_status_ != hipSuccess) {                           \
      return ::lcr::capi::hip_failure(#expr, capi_status_);     \
    }                                                           \
  } while (0)

// After a kernel launch: report a launch failure, and synchronize when
// LCR_SYNC_KERNELS=1 so a fault is attributed to this launch.
#define CAPI_LAUNCHED()                                                     \
  do {                                                                      \
    CAPI_HIP(hipGetLastError());                                            \
    if (::lcr::synchronous_launches()) CAPI_HIP(hipDeviceSynchronize());    \
  } while (0)
