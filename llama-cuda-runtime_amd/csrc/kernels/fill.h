// Device-side table and buffer fills:
//  - seeded N(0, stddev^2) elements, for the long-context stress case whose
//    cache is pre-filled rather than prefilled;
//  - the rotation table of the fused decode step: entry p * half + i holds
//    (cos, sin) of float(p) * inv_freq[i], computed by lcr_sincosf from the
//    very same float angle the RoPE kernels form, so a lookup equals the
//    computation bit for bit.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../dtype.h"

namespace lcr {

void fill_normal(elem_t* data, size_t count, uint64_t seed, float stddev, hipStream_t stream);

void build_rope_table(float2* table, const float* inv_freq, int positions, int half,
                      hipStream_t stream);

}  // namespace lcr
