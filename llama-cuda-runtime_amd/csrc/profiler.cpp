#include "profiler.h"

#include <algorithm>
#include <numeric>

#include "hip_utils.h"

namespace lcr {

Profiler::~Profiler() {
  for (hipEvent_t e : events_) (void)hipEventDestroy(e);
}

hipEvent_t Profiler::stamp_event() {
  const size_t slot = timeline_.size();
  while (events_.size() <= slot) {
    hipEvent_t e = nullptr;
    HIP_CHECK(hipEventCreate(&e));
    events_.push_back(e);
  }
  return events_[slot];
}

int Profiler::intern(const std::string& name) {
  const auto found = index_.find(name);
  if (found != index_.end()) return found->second;
  const int id = static_cast<int>(names_.size());
  names_.push_back(name);
  stage_ms_.push_back(0.0);
  stage_count_.push_back(0);
  index_.emplace(name, id);
  return id;
}

void Profiler::begin(const std::string& name, hipStream_t stream) {
  LCR_CHECK(timeline_.empty() || timeline_.back().stage < 0,
            "profiler stage \"" << name << "\" opened inside \"" << names_[timeline_.back().stage] << "\"");
  const Stamp s{intern(name), stamp_event()};
  HIP_CHECK(hipEventRecord(s.event, stream));
  timeline_.push_back(s);
}

void Profiler::end(hipStream_t stream) {
  LCR_CHECK(!timeline_.empty() && timeline_.back().stage >= 0, "profiler end() with no open stage");
  const Stamp s{-1, stamp_event()};
  HIP_CHECK(hipEventRecord(s.event, stream));
  timeline_.push_back(s);
}

void Profiler::collect() {
  if (timeline_.empty()) return;
  HIP_CHECK(hipEventSynchronize(timeline_.back().event));
  // Stamps alternate open, close; an open stage left at the end is dropped.
  for (size_t i = 0; i + 1 < timeline_.size(); i += 2) {
    const Stamp& open = timeline_[i];
    const Stamp& close = timeline_[i + 1];
    float ms = 0.0f;
    HIP_CHECK(hipEventElapsedTime(&ms, open.event, close.event));
    stage_ms_[static_cast<size_t>(open.stage)] += ms;
    stage_count_[static_cast<size_t>(open.stage)] += 1;
  }
  timeline_.clear();
}

std::vector<Profiler::Entry> Profiler::entries() const {
  std::vector<Entry> out;
  for (size_t i = 0; i < names_.size(); ++i) {
    if (stage_count_[i] > 0) out.push_back(Entry{names_[i], stage_ms_[i], stage_count_[i]});
  }
  std::stable_sort(out.begin(), out.end(),
                   [](const Entry& a, const Entry& b) { return a.total_ms > b.total_ms; });
  return out;
}

double Profiler::total_ms() const { return std::accumulate(stage_ms_.begin(), stage_ms_.end(), 0.0); }

int Profiler::total_launches() const {
  return std::accumulate(stage_count_.begin(), stage_count_.end(), 0);
}

void Profiler::reset() {
  timeline_.clear();
  std::fill(stage_ms_.begin(), stage_ms_.end(), 0.0);
  std::fill(stage_count_.begin(), stage_count_.end(), 0);
}

}  // namespace lcr
