// Seeded normal fill: element i of the buffer comes from pair i/2 of a
// counter-based stream (splitmix64 of seed and pair index, two 32-bit
// uniforms, Box-Muller), so the content depends only on (seed, i) and not on
// the launch shape.
#include <algorithm>

#include "../hip_utils.h"
#include "device_common.h"
#include "fill.h"

namespace lcr {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(elem_t* __restrict__ data, size_t count, uint64_t seed,
                                   float stddev) {
  const size_t pairs = (count + 1) / 2;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t p = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < pairs; p += stride) {
    const uint64_t h = mix64(seed * 0x9e3779b97f4a7c15ull + p);
    const float u1 = (static_cast<float>(static_cast<uint32_t>(h >> 40)) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = static_cast<float>(static_cast<uint32_t>(h & 0xffffffu)) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * logf(u1)) * stddev;
    float s, c;
    sincosf(6.28318530717958647692f * u2, &s, &c);
    data[2 * p] = float_to_elem(r * c);
    if (2 * p + 1 < count) data[2 * p + 1] = float_to_elem(r * s);
  }
}

__global__ void rope_table_kernel(float2* __restrict__ table, const float* __restrict__ inv_freq,
                                  int positions, int half) {
  const size_t n = static_cast<size_t>(positions) * half;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t e = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n; e += stride) {
    const int p = static_cast<int>(e / half);
    const int i = static_cast<int>(e % half);
    float s, c;
    lcr_sincosf(static_cast<float>(p) * inv_freq[i], &s, &c);
    table[e] = make_float2(c, s);
  }
}

}  // namespace

void build_rope_table(float2* table, const float* inv_freq, int positions, int half,
                      hipStream_t stream) {
  const size_t n = static_cast<size_t>(positions) * half;
  if (n == 0) return;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((n + 255) / 256, 4096));
  rope_table_kernel<<<blocks, 256, 0, stream>>>(table, inv_freq, positions, half);
  HIP_CHECK_LAUNCH();
}

void fill_normal(elem_t* data, size_t count, uint64_t seed, float stddev, hipStream_t stream) {
  if (count == 0) return;
  const size_t pairs = (count + 1) / 2;
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((pairs + 255) / 256, 16384));
  fill_normal_kernel<<<blocks, 256, 0, stream>>>(data, count, seed, stddev);
  HIP_CHECK_LAUNCH();
}

}  // namespace lcr
