#include "profiler.h"

#include <algorithm>

#include "hip_utils.h"

namespace lcr {

Profiler::~Profiler() {
  for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
}

hipEvent_t Profiler::acquire_event() {
  if (pool_used_ == pool_.size()) {
    hipEvent_t e;
    HIP_CHECK(hipEventCreate(&e));
    pool_.push_back(e);
  }
  return pool_[pool_used_++];
}

void Profiler::begin(const std::string& name, hipStream_t stream) {
  Span span;
  span.name = name;
  span.start = acquire_event();
  span.stop = nullptr;
  HIP_CHECK(hipEventRecord(span.start, stream));
  spans_.push_back(span);
}

void Profiler::end(hipStream_t stream) {
  LCR_CHECK(!spans_.empty() && spans_.back().stop == nullptr, "profiler end without begin");
  spans_.back().stop = acquire_event();
  HIP_CHECK(hipEventRecord(spans_.back().stop, stream));
}

void Profiler::collect() {
  for (const Span& span : spans_) {
    if (span.stop == nullptr) continue;
    HIP_CHECK(hipEventSynchronize(span.stop));
    float ms = 0.0f;
    HIP_CHECK(hipEventElapsedTime(&ms, span.start, span.stop));
    Entry& e = totals_[span.name];
    e.name = span.name;
    e.total_ms += ms;
    e.launches += 1;
  }
  spans_.clear();
  pool_used_ = 0;
}

std::vector<Profiler::Entry> Profiler::entries() const {
  std::vector<Entry> out;
  for (const auto& kv : totals_) out.push_back(kv.second);
  std::sort(out.begin(), out.end(), [](const Entry& a, const Entry& b) { return a.total_ms > b.total_ms; });
  return out;
}

double Profiler::total_ms() const {
  double t = 0.0;
  for (const auto& kv : totals_) t += kv.second.total_ms;
  return t;
}

int Profiler::total_launches() const {
  int n = 0;
  for (const auto& kv : totals_) n += kv.second.launches;
  return n;
}

void Profiler::reset() {
  totals_.clear();
  spans_.clear();
  pool_used_ = 0;
}

}  // namespace lcr
