// HIP status checks, the device description the token loop plans with, and a
// stream-region timer.
//
// Names kept from the reference's src/cuda_utils.cuh:21-89 so that host code
// ports unchanged: HIP_CHECK, HIP_CHECK_LAUNCH, synchronous_launches()
// (LCR_SYNC_KERNELS=1 synchronizes after every launch, so a fault surfaces at
// the launch that caused it), DeviceInfo / query_device and GpuTimer.
//
// DeviceInfo describes a CDNA device the way the kernels are planned: compute
// units and how many XCDs (each with its own L2) they are split over, the
// wavefront width, LDS per workgroup, and the HBM peak. The peak is the
// published figure for the architectures listed in hip_utils.cpp (MI355X:
// 8.0 TB/s) and otherwise 2 x memory clock x bus width from the properties.
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <type_traits>

#include "common.h"

namespace lcr {

namespace detail {
[[noreturn]] void fail_hip(hipError_t status, const char* call, const char* file, int line);

inline void check_hip(hipError_t status, const char* call, const char* file, int line) {
  if (status != hipSuccess) fail_hip(status, call, file, line);
}

// Called after a kernel launch: launch errors, and the optional synchronize.
void check_launch(const char* file, int line);
}  // namespace detail

#define HIP_CHECK(expr) ::lcr::detail::check_hip((expr), #expr, __FILE__, __LINE__)
#define HIP_CHECK_LAUNCH() ::lcr::detail::check_launch(__FILE__, __LINE__)

// True when LCR_SYNC_KERNELS is set to a value other than "" or "0".
bool synchronous_launches();

struct DeviceInfo {
  int index = 0;
  std::string name;
  std::string arch;              // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
  int multiprocessors = 0;       // compute units
  int xcds = 1;                  // accelerator complex dies (one L2 each)
  int wavefront_size = 64;
  size_t lds_bytes_per_block = 0;
  size_t total_memory = 0;
  int memory_bus_width_bits = 0;
  int memory_clock_khz = 0;
  int l2_cache_bytes = 0;        // per XCD, as the runtime reports it
  double published_peak_bytes_per_second = 0.0;  // 0 when the arch is not tabulated

  // HBM peak the benchmark divides by: the published figure when known,
  // otherwise derived from the memory clock and bus width.
  double peak_bandwidth_bytes_per_second() const;
  double derived_peak_bandwidth_bytes_per_second() const;
  // True when arch names gfx950 (MI350X / MI355X).
  bool is_gfx950() const;
  std::string summary() const;
};

DeviceInfo query_device(int index);

// Times a region of a stream with two events; the host only waits in
// elapsed_ms().
class GpuTimer {
 public:
  GpuTimer();
  void start(hipStream_t stream = nullptr);
  void stop(hipStream_t stream = nullptr);
  double elapsed_ms() const;

 private:
  struct EventDeleter {
    void operator()(std::remove_pointer_t<hipEvent_t>* e) const { (void)hipEventDestroy(e); }
  };
  using EventHandle = std::unique_ptr<std::remove_pointer_t<hipEvent_t>, EventDeleter>;
  static EventHandle make_event();

  EventHandle begin_;
  EventHandle end_;
};

}  // namespace lcr
