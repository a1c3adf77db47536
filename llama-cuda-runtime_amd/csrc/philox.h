// Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC 2011): the counter-based generator of the sampling
// draws. Draw i of seed s is word i % 4 of Philox(counter = (i / 4, 0, 0, 0),
// key = (s low, s high)), mapped to [0, 1) as (word >> 8) * 2^-24, which is
// exact in float32; the same stream the tests feed the CPU oracle's sampler.
#pragma once

#include <array>
#include <cstdint>

namespace lcr {

inline std::array<uint32_t, 4> philox4x32_10(std::array<uint32_t, 4> c, std::array<uint32_t, 2> k) {
  for (int round = 0; round < 10; ++round) {
    const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c[0];
    const uint64_t p1 = static_cast<uint64_t>(0xCD9E8D57u) * c[2];
    c = {static_cast<uint32_t>(p1 >> 32) ^ c[1] ^ k[0], static_cast<uint32_t>(p1),
         static_cast<uint32_t>(p0 >> 32) ^ c[3] ^ k[1], static_cast<uint32_t>(p0)};
    k = {k[0] + 0x9E3779B9u, k[1] + 0xBB67AE85u};
  }
  return c;
}

class PhiloxUniforms {
 public:
  explicit PhiloxUniforms(uint64_t seed)
      : key_{static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32)} {}
  float next() {
    if (index_ % 4 == 0) block_ = philox4x32_10({static_cast<uint32_t>(index_ / 4), 0, 0, 0}, key_);
    const uint32_t word = block_[index_ % 4];
    ++index_;
    return static_cast<float>(word >> 8) * (1.0f / 16777216.0f);
  }

 private:
  std::array<uint32_t, 2> key_;
  std::array<uint32_t, 4> block_{};
  uint64_t index_ = 0;
};

}  // namespace lcr
