// Per-stage event timing of a forward pass (drop-in for the reference's
// src/profiler.h:25-87): a pair of pooled hipEvents around each named stage,
// accumulated by name. Stage timing needs eager launches, so it applies to
// the unfused path; the fused, graph-captured decode step is measured with
// rocprofv3 instead.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace lcr {

class Profiler {
 public:
  ~Profiler();

  void set_enabled(bool enabled) { enabled_ = enabled; }
  bool enabled() const { return enabled_; }

  void begin(const std::string& name, hipStream_t stream);
  void end(hipStream_t stream);
  // Waits for the recorded events and folds them into the totals.
  void collect();

  struct Entry {
    std::string name;
    double total_ms = 0.0;
    int launches = 0;
  };
  std::vector<Entry> entries() const;  // by total time, descending
  double total_ms() const;
  int total_launches() const;
  void reset();

 private:
  struct Span {
    std::string name;
    hipEvent_t start;
    hipEvent_t stop;
  };
  hipEvent_t acquire_event();

  bool enabled_ = false;
  std::vector<Span> spans_;
  std::vector<hipEvent_t> pool_;
  size_t pool_used_ = 0;
  std::unordered_map<std::string, Entry> totals_;
};

class ProfileScope {
 public:
  ProfileScope(Profiler* profiler, const char* name, hipStream_t stream)
      : profiler_(profiler), stream_(stream) {
    if (profiler_ != nullptr && profiler_->enabled()) {
      profiler_->begin(name, stream_);
      active_ = true;
    }
  }
  ~ProfileScope() {
    if (active_) profiler_->end(stream_);
  }
  ProfileScope(const ProfileScope&) = delete;
  ProfileScope& operator=(const ProfileScope&) = delete;

 private:
  Profiler* profiler_;
  hipStream_t stream_;
  bool active_ = false;
};

}  // namespace lcr
