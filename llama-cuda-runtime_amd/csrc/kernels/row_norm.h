// The row sum of squares behind every RMSNorm, in one fixed order.
//
// A 256-thread block reduces one row. Thread t squares-and-accumulates the
// 8-element chunks t, t+256, t+512, ... (elements in order, s = fma(v, v, s)),
// then the elements past the last whole chunk at positions t, t+256, ...; the
// 256 partials are added by a butterfly inside each aligned group of 32 threads
// (offsets 16..1), and the 8 group totals by the same 32-wide butterfly with
// zeros in lanes 8..31. That is the shape of the reference's rmsnorm kernels
// (src/kernels/rmsnorm.cu:32-47 with block_reduce_sum, reduce.cuh:23-37), so the
// order is well defined and the CPU oracle reproduces it exactly.
//
// The scale is 1 / sqrt(total / dim + eps) with a correctly rounded divide and
// square root, and each output is rne((x * scale) * w).
#pragma once

#include "device_common.h"

namespace lcr {

constexpr int kNormThreads = 256;

// Adds the per-thread partial sums of a 256-thread block in the fixed tree.
// Every thread must call it; every thread gets the total. `scratch` holds at
// least 8 floats of LDS. The second butterfly runs over the 8 group totals
// p0..p7 with zeros in lanes 8..31, where offsets 16 and 8 add nothing, so
// every thread evaluates its offsets 4, 2, 1 directly:
// ((p0 + p4) + (p2 + p6)) + ((p1 + p5) + (p3 + p7)).
// This form leaves `scratch` in use: the caller passes a barrier before it
// writes `scratch` again.
__device__ __forceinline__ float block_norm_total_once(float s, float* scratch) {
  const int t = static_cast<int>(threadIdx.x);
  s = half_wave_sum(s);
  if ((t & 31) == 0) scratch[t >> 5] = s;
  __syncthreads();
  return ((scratch[0] + scratch[4]) + (scratch[2] + scratch[6])) +
         ((scratch[1] + scratch[5]) + (scratch[3] + scratch[7]));
}

__device__ __forceinline__ float block_norm_total(float s, float* scratch) {
  const float total = block_norm_total_once(s, scratch);
  __syncthreads();
  return total;
}

// `get(i)` returns element i of the row as float; every thread of a
// 256-thread block must call this.
template <typename Get>
__device__ __forceinline__ float block_sum_squares(Get get, int dim, float* scratch) {
  const int t = static_cast<int>(threadIdx.x);
  float s = 0.0f;
  const int chunks = dim / 8;
  for (int c = t; c < chunks; c += kNormThreads) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = get(8 * c + j);
      s = __builtin_fmaf(v, v, s);
    }
  }
  for (int i = chunks * 8 + t; i < dim; i += kNormThreads) {
    const float v = get(i);
    s = __builtin_fmaf(v, v, s);
  }
  return block_norm_total(s, scratch);
}

__device__ __forceinline__ float norm_scale(float total, int dim, float eps) {
  return 1.0f / __builtin_sqrtf(total / static_cast<float>(dim) + eps);
}

// One row of RMSNorm (kResidual: of the residual add x += delta first) with
// 16-byte accesses and the row in registers, for rows of dim = 8 * chunks
// elements with at most kChunks chunks per thread: thread t holds chunks
// t, t + 256, ... (the order block_sum_squares walks), so the sum of squares
// and the roundings are those of block_sum_squares' element loop, bit for bit.
// delta(c, df) writes the eight addends of chunk c to df[0..7].
template <bool kResidual, int kChunks, typename Delta>
__device__ __forceinline__ void norm_row_vec(elem_t* __restrict__ orow, elem_t* __restrict__ xrow,
                                             const elem_t* __restrict__ weight, int dim, float eps,
                                             Delta delta, float* scratch) {
  const int chunks = dim / 8;
  const int t = static_cast<int>(threadIdx.x);
  float v[kChunks][8];
  vec16 w[kChunks];
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int c = t + k * kNormThreads;
    if (c >= chunks) continue;
    const vec16 xv = load16(xrow + 8 * c);
    w[k] = load16(weight + 8 * c);
    float xf[8];
    unpack8(xv, xf);
    if (kResidual) {
      float df[8];
      delta(c, df);
      vec16 r;
#pragma unroll
      for (int j = 0; j < 8; ++j) v[k][j] = xf[j] + df[j];
#pragma unroll
      for (int j = 0; j < 4; ++j) r.w[j] = pack_elems(v[k][2 * j], v[k][2 * j + 1]);
      store16(xrow + 8 * c, r);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[k][j] = xf[j];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s = __builtin_fmaf(v[k][j], v[k][j], s);
  }
  const float scale = norm_scale(block_norm_total(s, scratch), dim, eps);
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    const int c = t + k * kNormThreads;
    if (c >= chunks) continue;
    float wf[8];
    unpack8(w[k], wf);
    vec16 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = elem_bits_to_float(float_to_elem_bits(v[k][2 * j]));
      const float b = elem_bits_to_float(float_to_elem_bits(v[k][2 * j + 1]));
      r.w[j] = pack_elems((a * scale) * wf[2 * j], (b * scale) * wf[2 * j + 1]);
    }
    store16(orow + 8 * c, r);
  }
}

}  // namespace lcr
