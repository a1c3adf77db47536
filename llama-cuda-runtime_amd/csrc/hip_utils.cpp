#include "hip_utils.h"

#include <cstdlib>
#include <cstring>
#include <sstream>

namespace lcr {

namespace detail {

void fail_hip(hipError_t status, const char* call, const char* file, int line) {
  std::ostringstream text;
  text << hipGetErrorName(status) << " (" << hipGetErrorString(status) << ") from " << call
       << " [" << file << ":" << line << "]";
  throw Error(text.str());
}

void check_launch(const char* file, int line) {
  check_hip(hipGetLastError(), "kernel launch", file, line);
  if (synchronous_launches()) check_hip(hipDeviceSynchronize(), "hipDeviceSynchronize after launch", file, line);
}

}  // namespace detail

bool synchronous_launches() {
  static const bool on = [] {
    const char* value = std::getenv("LCR_SYNC_KERNELS");
    return value != nullptr && value[0] != '\0' && std::strcmp(value, "0") != 0;
  }();
  return on;
}

namespace {

// Published HBM peaks by architecture prefix.
struct PublishedPeak {
  const char* arch_prefix;
  double bytes_per_second;
};
constexpr PublishedPeak kPublishedPeaks[] = {
    {"gfx950", 8.0e12},  // MI350X / MI355X, HBM3E
    {"gfx942", 5.3e12},  // MI300X
};

double published_peak(const std::string& arch) {
  for (const PublishedPeak& p : kPublishedPeaks) {
    if (arch.compare(0, std::strlen(p.arch_prefix), p.arch_prefix) == 0) return p.bytes_per_second;
  }
  return 0.0;
}

}  // namespace

double DeviceInfo::derived_peak_bandwidth_bytes_per_second() const {
  // Double data rate: two transfers per memory clock across the bus.
  const double bus_bytes = memory_bus_width_bits / 8.0;
  return 2.0 * (memory_clock_khz * 1e3) * bus_bytes;
}

double DeviceInfo::peak_bandwidth_bytes_per_second() const {
  return published_peak_bytes_per_second > 0.0 ? published_peak_bytes_per_second
                                               : derived_peak_bandwidth_bytes_per_second();
}

bool DeviceInfo::is_gfx950() const { return arch.compare(0, 6, "gfx950") == 0; }

std::string DeviceInfo::summary() const {
  std::ostringstream text;
  text << name << " [" << arch << "] " << multiprocessors << " CUs on " << xcds << " XCDs, wave"
       << wavefront_size << ", " << format_bytes(total_memory) << " HBM, "
       << peak_bandwidth_bytes_per_second() / 1e12 << " TB/s peak ("
       << (published_peak_bytes_per_second > 0.0 ? "published" : "clock x bus") << ")";
  return text.str();
}

DeviceInfo query_device(int index) {
  int count = 0;
  HIP_CHECK(hipGetDeviceCount(&count));
  LCR_CHECK(count > 0, "no HIP device is visible");
  LCR_CHECK(index >= 0 && index < count,
            "requested device " << index << " but only " << count << " are visible");
  hipDeviceProp_t p{};
  HIP_CHECK(hipGetDeviceProperties(&p, index));
  DeviceInfo d;
  d.index = index;
  d.name = p.name;
  d.arch = p.gcnArchName;
  d.multiprocessors = p.multiProcessorCount;
  d.wavefront_size = p.warpSize;
  d.lds_bytes_per_block = p.sharedMemPerBlock;
  d.total_memory = p.totalGlobalMem;
  d.memory_bus_width_bits = p.memoryBusWidth;
  d.memory_clock_khz = p.memoryClockRate;
  d.l2_cache_bytes = p.l2CacheSize;
  int xcc = 0;
  if (hipDeviceGetAttribute(&xcc, hipDeviceAttributeNumberOfXccs, index) == hipSuccess && xcc > 0) {
    d.xcds = xcc;
  }
  d.published_peak_bytes_per_second = published_peak(d.arch);
  return d;
}

GpuTimer::EventHandle GpuTimer::make_event() {
  hipEvent_t e = nullptr;
  HIP_CHECK(hipEventCreate(&e));
  return EventHandle(e);
}

GpuTimer::GpuTimer() : begin_(make_event()), end_(make_event()) {}

void GpuTimer::start(hipStream_t stream) { HIP_CHECK(hipEventRecord(begin_.get(), stream)); }

void GpuTimer::stop(hipStream_t stream) { HIP_CHECK(hipEventRecord(end_.get(), stream)); }

double GpuTimer::elapsed_ms() const {
  HIP_CHECK(hipEventSynchronize(end_.get()));
  float ms = 0.0f;
  HIP_CHECK(hipEventElapsedTime(&ms, begin_.get(), end_.get()));
  return ms;
}

}  // namespace lcr
