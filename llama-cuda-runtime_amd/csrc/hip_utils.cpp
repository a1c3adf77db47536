#include "hip_utils.h"

#include <cstdlib>
#include <sstream>

namespace lcr {
namespace detail {

void throw_hip_error(const char* file, int line, const char* expr, hipError_t status) {
  std::ostringstream oss;
  oss << file << ":" << line << ": HIP call failed: " << expr << "\n  "
      << hipGetErrorName(status) << ": " << hipGetErrorString(status);
  throw Error(oss.str());
}

}  // namespace detail

bool synchronous_launches() {
  static const bool enabled = [] {
    const char* v = std::getenv("LCR_SYNC_KERNELS");
    return v != nullptr && v[0] == '1';
  }();
  return enabled;
}

double DeviceInfo::peak_bandwidth_bytes_per_second() const {
  return 2.0 * static_cast<double>(memory_clock_khz) * 1000.0 *
         (static_cast<double>(memory_bus_width_bits) / 8.0);
}

std::string DeviceInfo::summary() const {
  std::ostringstream oss;
  oss << name << " (" << arch << ", " << multiprocessors << " CUs, "
      << format_bytes(total_memory) << ", " << memory_bus_width_bits << "-bit bus, "
      << peak_bandwidth_bytes_per_second() / 1e9 << " GB/s peak)";
  return oss.str();
}

DeviceInfo query_device(int index) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  LCR_CHECK(count > 0, "no HIP device is visible");
  LCR_CHECK(index >= 0 && index < count,
            "requested device " << index << " but only " << count << " are visible");
  hipDeviceProp_t props{};
  HIP_CHECK(hipGetDeviceProperties(&props, index));
  DeviceInfo info;
  info.index = index;
  info.name = props.name;
  info.arch = props.gcnArchName;
  info.multiprocessors = props.multiProcessorCount;
  info.total_memory = props.totalGlobalMem;
  info.memory_bus_width_bits = props.memoryBusWidth;
  info.memory_clock_khz = props.memoryClockRate;
  info.l2_cache_bytes = props.l2CacheSize;
  return info;
}

GpuTimer::GpuTimer() {
  HIP_CHECK(hipEventCreate(&start_));
  HIP_CHECK(hipEventCreate(&stop_));
}

GpuTimer::~GpuTimer() {
  (void)hipEventDestroy(start_);
  (void)hipEventDestroy(stop_);
}

void GpuTimer::start(hipStream_t stream) { HIP_CHECK(hipEventRecord(start_, stream)); }
void GpuTimer::stop(hipStream_t stream) { HIP_CHECK(hipEventRecord(stop_, stream)); }

double GpuTimer::elapsed_ms() const {
  HIP_CHECK(hipEventSynchronize(stop_));
  float ms = 0.0f;
  HIP_CHECK(hipEventElapsedTime(&ms, start_, stop_));
  return ms;
}

}  // namespace lcr
