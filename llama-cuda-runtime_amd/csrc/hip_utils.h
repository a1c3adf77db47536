// HIP error checking, device properties and event timing.
//
// The host-side conventions of the reference's src/cuda_utils.cuh:21-89:
// HIP_CHECK throws lcr::Error naming the failed call, HIP_CHECK_LAUNCH checks
// the launch and, with LCR_SYNC_KERNELS=1, synchronizes after it so a fault is
// reported at the launch that caused it. DeviceInfo reports the peak HBM
// bandwidth the benchmark divides by; GpuTimer brackets a stream region with
// two events.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "common.h"

namespace lcr {

namespace detail {
[[noreturn]] void throw_hip_error(const char* file, int line, const char* expr,
                                  hipError_t status);
}  // namespace detail

#define HIP_CHECK(expr)                                                        \
  do {                                                                         \
    const hipError_t lcr_hip_status_ = (expr);                                 \
    if (lcr_hip_status_ != hipSuccess) {                                       \
      ::lcr::detail::throw_hip_error(__FILE__, __LINE__, #expr, lcr_hip_status_); \
    }                                                                          \
  } while (0)

#define HIP_CHECK_LAUNCH()                                                     \
  do {                                                                         \
    HIP_CHECK(hipGetLastError());                                              \
    if (::lcr::synchronous_launches()) HIP_CHECK(hipDeviceSynchronize());      \
  } while (0)

// LCR_SYNC_KERNELS=1: synchronize after every launch.
bool synchronous_launches();

struct DeviceInfo {
  int index = 0;
  std::string name;
  std::string arch;
  int multiprocessors = 0;
  size_t total_memory = 0;
  int memory_bus_width_bits = 0;
  int memory_clock_khz = 0;
  int l2_cache_bytes = 0;

  // 2 x memory clock x bus width: for MI355X 2 x 2.0 GHz x 8192 bit = 8.19 TB/s
  // (the published figure is 8.0 TB/s; the benchmark reports which it used).
  double peak_bandwidth_bytes_per_second() const;
  std::string summary() const;
};

DeviceInfo query_device(int index);

class GpuTimer {
 public:
  GpuTimer();
  ~GpuTimer();
  GpuTimer(const GpuTimer&) = delete;
  GpuTimer& operator=(const GpuTimer&) = delete;

  void start(hipStream_t stream = nullptr);
  void stop(hipStream_t stream = nullptr);
  double elapsed_ms() const;  // waits for the stop event

 private:
  hipEvent_t start_{};
  hipEvent_t stop_{};
};

}  // namespace lcr
