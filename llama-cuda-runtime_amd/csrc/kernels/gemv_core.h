// Batch-1 matrix-vector product on one wavefront: the projection kernel of
// decode (the cuBLAS calls of the reference's src/model.cu:38-45 at rows = 1).
//
// Decode multiplies every weight exactly once, so the kernel is a weight
// stream: each lane issues 16-byte loads, one row of K = 2048 bf16 is 64 lanes
// x 64 bytes, and every load of a row is in flight before the first multiply.
// No matrix cores: a matrix-vector product has nothing for them to reuse.
//
// Summation order (fixed; the CPU oracle repeats it exactly):
//  - the row is cut into blocks of 2048 elements (the last one may be short);
//  - inside a block, lane l owns the 8-element chunks l, l+64, l+128, l+192
//    of the block and accumulates them in that order, element by element,
//    acc = fma(w, x, acc) starting from +0 (chunks past the end of the row
//    are skipped, not multiplied by zero);
//  - the block sum is the butterfly over the 64 lanes (offsets 32..1);
//  - the row sum is block0 + block1 + ... from left to right.
#pragma once

#include "device_common.h"

namespace lcr {

constexpr int kGemvChunk = 8;          // elements per 16-byte load
constexpr int kGemvBlock = 2048;       // elements per reduction block
constexpr int kGemvLaneChunks = kGemvBlock / (64 * kGemvChunk);  // 4

// fma of one 16-byte weight chunk against one 16-byte x chunk, in element order.
__device__ __forceinline__ float dot_chunk(const vec16& w, const vec16& x, float acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = __builtin_fmaf(elem_lo(w.w[i]), elem_lo(x.w[i]), acc);
    acc = __builtin_fmaf(elem_hi(w.w[i]), elem_hi(x.w[i]), acc);
  }
  return acc;
}

// R rows of a matrix whose K is a multiple of 2048, NCH = K / 512 chunks per
// lane. `rows[r]` are row pointers (already offset to the row start).
template <int R, int NCH>
struct GemvTile {
  vec16 w[R][NCH];

  __device__ __forceinline__ void load(const elem_t* const (&rows)[R], int lane) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) w[r][c] = load16_stream(rows[r] + c * 512 + lane * kGemvChunk);
    }
  }

  // out[r] = full-row dot products in the fixed order; every lane gets them.
  __device__ __forceinline__ void dot(float (&out)[R], const vec16 (&x)[NCH]) const {
    static_assert(NCH % kGemvLaneChunks == 0, "K must be a multiple of 2048");
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float total = 0.0f;
#pragma unroll
      for (int b = 0; b < NCH / kGemvLaneChunks; ++b) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < kGemvLaneChunks; ++c) {
          acc = dot_chunk(w[r][b * kGemvLaneChunks + c], x[b * kGemvLaneChunks + c], acc);
        }
        const float s = wave_sum(acc);
        total = (b == 0) ? s : total + s;
      }
      out[r] = total;
    }
  }
};

// The same order for any K that is a multiple of 8, one block at a time
// (fewer loads in flight; used for shapes outside the model's).
__device__ __forceinline__ float gemv_row_generic(const elem_t* __restrict__ row,
                                                  const elem_t* __restrict__ x, int K, int lane) {
  float total = 0.0f;
  const int blocks = (K + kGemvBlock - 1) / kGemvBlock;
  for (int b = 0; b < blocks; ++b) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < kGemvLaneChunks; ++c) {
      const int e = b * kGemvBlock + c * 512 + lane * kGemvChunk;
      if (e < K) acc = dot_chunk(load16(row + e), load16(x + e), acc);
    }
    const float s = wave_sum(acc);
    total = (b == 0) ? s : total + s;
  }
  return total;
}

}  // namespace lcr
