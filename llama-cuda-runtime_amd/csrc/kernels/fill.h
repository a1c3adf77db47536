// Device-side fill of a buffer with seeded N(0, stddev^2) elements, for the
// long-context stress case whose cache is pre-filled rather than prefilled.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../dtype.h"

namespace lcr {

void fill_normal(elem_t* data, size_t count, uint64_t seed, float stddev, hipStream_t stream);

}  // namespace lcr
