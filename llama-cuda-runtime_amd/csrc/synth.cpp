// Seeded random-init checkpoints and prompts.
//
// There is no network, so no real Llama checkpoint: the GPU path and the CPU
// oracle both read a synthetic one written here, with the reference's tensor
// names and shapes (src/config.cpp:197-221) and the statistics the benchmark
// configurations name: every projection N(0, 0.02^2), every norm weight 1.0,
// tied embeddings. Element i of tensor t comes from a counter-based stream, so
// the bytes depend only on (seed, t, i):
//   base = mix(seed ^ 0xC2B2AE3D27D4EB4F * (t + 1))      (splitmix64 finaliser)
//   a = mix(base + 2p), b = mix(base + 2p + 1)            for pair p = i / 2
//   u1 = ((a >> 11) + 1) * 2^-53 in (0, 1], u2 = (b >> 11) * 2^-53 in [0, 1)
//   z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2)  (Box-Muller)
//   element 2p = rne16(float(z0 * std)), element 2p + 1 = rne16(float(z1 * std))
// Prompt ids are uniform in [0, vocab) by Lemire's multiply-shift of the high
// 32 bits of mix(seed * 0x9E3779B97F4A7C15 + i).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <fstream>
#include <string>
#include <sys/stat.h>
#include <thread>
#include <vector>

#include "capi_util.h"
#include "philox.h"
#include "config.h"
#include "dtype.h"
#include "safetensors.h"

namespace lcr {
namespace {

uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

bool is_norm(const std::string& name) {
  const std::string suffix = "norm.weight";
  return name.size() >= suffix.size() &&
         name.compare(name.size() - suffix.size(), suffix.size(), suffix) == 0;
}

void fill_tensor(uint16_t* dst, size_t count, uint64_t seed, size_t tensor, float stddev,
                 bool fp16, bool ones, int threads) {
  const uint16_t one = fp16 ? float_to_half_bits(1.0f) : float_to_bf16_bits(1.0f);
  if (ones) {
    std::fill(dst, dst + count, one);
    return;
  }
  const uint64_t base = mix64(seed ^ (0xC2B2AE3D27D4EB4Full * (tensor + 1)));
  const size_t pairs = (count + 1) / 2;
  auto work = [&](size_t begin, size_t end) {
    for (size_t p = begin; p < end; ++p) {
      const uint64_t a = mix64(base + 2 * p);
      const uint64_t b = mix64(base + 2 * p + 1);
      const double u1 = static_cast<double>((a >> 11) + 1) * 0x1.0p-53;
      const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;
      const double r = std::sqrt(-2.0 * std::log(u1));
      const double angle = 2.0 * M_PI * u2;
      const float z0 = static_cast<float>(r * std::cos(angle) * stddev);
      const float z1 = static_cast<float>(r * std::sin(angle) * stddev);
      dst[2 * p] = fp16 ? float_to_half_bits(z0) : float_to_bf16_bits(z0);
      if (2 * p + 1 < count) dst[2 * p + 1] = fp16 ? float_to_half_bits(z1) : float_to_bf16_bits(z1);
    }
  };
  const size_t n = static_cast<size_t>(std::max(1, threads));
  if (n == 1 || pairs < 65536) {
    work(0, pairs);
    return;
  }
  std::vector<std::thread> pool;
  const size_t per = (pairs + n - 1) / n;
  for (size_t t = 0; t < n; ++t) {
    const size_t b = std::min(pairs, t * per);
    const size_t e = std::min(pairs, b + per);
    if (b < e) pool.emplace_back(work, b, e);
  }
  for (std::thread& th : pool) th.join();
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" int lcr_write_synthetic_checkpoint(const char* dir, const char* config_json,
                                              uint64_t seed, float stddev, int fp16,
                                              int threads) {
  capi::clear_error();
  return capi::guarded([&]() -> int {
    CAPI_CHECK(dir != nullptr && config_json != nullptr, "checkpoint directory and config needed");
    const ModelConfig config = ModelConfig::from_json_string(config_json);
    ::mkdir(dir, 0755);
    const std::string d(dir);
    {
      std::ofstream out(d + "/config.json", std::ios::binary | std::ios::trunc);
      CAPI_CHECK(out.good(), "cannot write " << d << "/config.json");
      out << config_json;
    }
    std::vector<TensorSpec> specs;
    for (const WeightSpec& w : required_weights(config)) {
      specs.push_back({w.name, fp16 ? DType::kF16 : DType::kBF16, w.shape});
    }
    if (!config.tie_word_embeddings) {
      specs.push_back({"lm_head.weight", fp16 ? DType::kF16 : DType::kBF16,
                       {config.vocab_size, config.hidden_size}});
    }
    write_safetensors(d + "/model.safetensors", specs, [&](size_t index, void* dst, size_t nbytes) {
      fill_tensor(static_cast<uint16_t*>(dst), nbytes / 2, seed, index, stddev, fp16 != 0,
                  is_norm(specs[index].name), threads);
    });
    return LCR_OK;
  });
}

extern "C" int lcr_synthetic_tokens(uint64_t seed, int count, int vocab, int32_t* out) {
  capi::clear_error();
  CAPI_CHECK(count >= 0 && vocab > 0 && (count == 0 || out != nullptr),
             "synthetic tokens need a positive vocabulary and an output buffer");
  for (int i = 0; i < count; ++i) {
    const uint64_t h = mix64(seed * 0x9e3779b97f4a7c15ull + static_cast<uint64_t>(i));
    const uint64_t hi = h >> 32;
    out[i] = static_cast<int32_t>((hi * static_cast<uint64_t>(vocab)) >> 32);
  }
  return LCR_OK;
}

extern "C" int lcr_philox_uniforms(uint64_t seed, int count, float* out) {
  capi::clear_error();
  CAPI_CHECK(count >= 0 && (count == 0 || out != nullptr), "philox draws need an output buffer");
  PhiloxUniforms draws(seed);
  for (int i = 0; i < count; ++i) out[i] = draws.next();
  return LCR_OK;
}
