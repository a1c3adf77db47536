// Per-stage timing of an eager forward pass from hipEvents.
//
// Interface of the reference's Profiler / ProfileScope (src/profiler.h:25-87):
// set_enabled, begin / end around a stage, collect, entries sorted by time,
// total_ms, total_launches, reset. The design is a timeline: every begin and
// every end records one stamp (an event from a reusable pool, slot i for the
// i-th stamp of a pass), stage names are interned to indices, and collect()
// waits once, on the last stamp (a stream completes its events in order),
// before reading each stage's begin-to-end time. Stages do not nest.
//
// It applies to the unfused, eagerly launched path; the graph-captured decode
// step runs as one graph launch and is measured with rocprofv3 instead.
#pragma once

#include <hip/hip_runtime.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace lcr {

class Profiler {
 public:
  Profiler() = default;
  ~Profiler();
  Profiler(const Profiler&) = delete;
  Profiler& operator=(const Profiler&) = delete;

  void set_enabled(bool enabled) { enabled_ = enabled; }
  bool enabled() const { return enabled_; }

  void begin(const std::string& name, hipStream_t stream);
  void end(hipStream_t stream);
  // Waits for this pass's stamps and adds each stage's time to its total.
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
  struct Stamp {
    int stage;  // index into names_; -1 closes the stage opened before it
    hipEvent_t event;
  };
  hipEvent_t stamp_event();
  int intern(const std::string& name);

  bool enabled_ = false;
  std::vector<hipEvent_t> events_;  // pool; grows to the longest pass
  std::vector<Stamp> timeline_;     // this pass, in record order
  std::vector<std::string> names_;
  std::unordered_map<std::string, int> index_;
  std::vector<double> stage_ms_;
  std::vector<int> stage_count_;
};

// Opens a stage for the lifetime of the scope (when the profiler is enabled).
class ProfileScope {
 public:
  ProfileScope(Profiler* profiler, const char* name, hipStream_t stream)
      : profiler_(profiler != nullptr && profiler->enabled() ? profiler : nullptr), stream_(stream) {
    if (profiler_ != nullptr) profiler_->begin(name, stream_);
  }
  ~ProfileScope() {
    if (profiler_ != nullptr) profiler_->end(stream_);
  }
  ProfileScope(const ProfileScope&) = delete;
  ProfileScope& operator=(const ProfileScope&) = delete;

 private:
  Profiler* const profiler_;
  hipStream_t stream_;
};

}  // namespace lcr
