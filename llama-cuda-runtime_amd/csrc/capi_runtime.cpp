// Device memory helpers of include/lcr_runtime.h.
#include "../../include/lcr_runtime.h"

#include "capi_util.h"

using namespace lcr;

extern "C" int lcr_device_malloc(void** out, size_t bytes) {
  capi::clear_error();
  CAPI_CHECK(out != nullptr, "device_malloc needs an output pointer");
  *out = nullptr;
  if (bytes == 0) return LCR_OK;
  CAPI_HIP(hipMalloc(out, bytes));
  return LCR_OK;
}

extern "C" int lcr_device_free(void* ptr) {
  capi::clear_error();
  if (ptr == nullptr) return LCR_OK;
  CAPI_HIP(hipFree(ptr));
  return LCR_OK;
}

extern "C" int lcr_memcpy_htod(void* dst, const void* src, size_t bytes) {
  capi::clear_error();
  if (bytes == 0) return LCR_OK;
  CAPI_HIP(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  return LCR_OK;
}

extern "C" int lcr_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
  capi::clear_error();
  if (bytes == 0) return LCR_OK;
  CAPI_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return LCR_OK;
}

extern "C" int lcr_memcpy_dtod(void* dst, const void* src, size_t bytes) {
  capi::clear_error();
  if (bytes == 0) return LCR_OK;
  CAPI_HIP(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
  return LCR_OK;
}

extern "C" int lcr_device_memset(void* ptr, int value, size_t bytes) {
  capi::clear_error();
  if (bytes == 0) return LCR_OK;
  CAPI_HIP(hipMemset(ptr, value, bytes));
  return LCR_OK;
}

extern "C" int lcr_device_synchronize(void) {
  capi::clear_error();
  CAPI_HIP(hipDeviceSynchronize());
  return LCR_OK;
}
