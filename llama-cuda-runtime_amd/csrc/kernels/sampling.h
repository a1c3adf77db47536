// Token selection from fp32 logits, shared by the launcher and the fused
// decode step.
//
// Greedy: argmax with ties to the lowest index, via the packed 64-bit key of
// the reference (src/kernels/sampling.cu:37-61): (order-preserving 32-bit key
// of the logit) << 32 | (0xFFFFFFFF - index). The maximum key is unique and
// order-independent, so any reduction tree gives the same id. Here it is two
// passes without atomics: blocks write their maximum to scratch, one block
// reduces those and writes the id, so there is nothing to clear between calls.
//
// Stochastic: the reference's one-block sampler (sampling.cu:97-224) with its
// two scheduling-dependent steps made deterministic, spread over kernels
// without changing a result: the argmax blocks' partial maxima (step 1);
// sixteen one-wave blocks that each run 64 threads of the 1024-thread order
// below and write their partial sums and bin counts (step 2); one block per
// 1024 logits that finds the cutoff (step 3) and writes its candidates in
// index order (step 4); one 1024-thread block for step 2's final sum, the
// first 1024 candidates in block order, the sort and the walk (5-6):
//  1. max logit (exact), scaled_i = (l_i - max) * inv_temperature;
//  2. total = sum of exp(scaled_i): thread t (of 1024) adds i = t, t+1024, ...
//     in order, then a butterfly in each 32-thread group (offsets 16..1), then
//     the 32 group sums by the same butterfly (the reference's
//     block_reduce_sum order); histogram of bin = min(255, int(-scaled*12.8));
//  3. cutoff bin = deepest bin whose running count stays <= 1024 (at least 1);
//  4. candidates (bin < cutoff) are compacted in increasing index order — the
//     reference uses an atomic counter, whose order varies from run to run;
//  5. candidates are sorted by (scaled value descending, index ascending) — a
//     total order, where the reference's bitonic sort leaves equal values in
//     arbitrary order;
//  6. one thread walks the sorted list exactly as the reference does:
//     kept_mass = fma(exp(v_i), 1/total, kept_mass) up to top_k, stopping at
//     the first i where top_p < 1 and kept_mass >= top_p (that token kept);
//     then target = uniform * kept_mass and the first i with
//     running = fma(exp(v_i), 1/total, running) >= target is the sample.
#pragma once

#include <hip/hip_runtime.h>

#include "device_common.h"

namespace lcr {

constexpr int kArgmaxBlocks = 256;
constexpr int kArgmaxThreads = 256;
constexpr int kSampleThreads = 1024;
constexpr int kMaxCandidates = 1024;
constexpr int kHistogramBins = 256;

__host__ __device__ __forceinline__ uint32_t order_key(float value) {
  const uint32_t bits = f32_as_u32(value);
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

__host__ __device__ __forceinline__ unsigned long long argmax_key(float value, uint32_t index) {
  return (static_cast<unsigned long long>(order_key(value)) << 32) |
         static_cast<unsigned long long>(0xFFFFFFFFu - index);
}

__device__ __forceinline__ unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

template <int O>
__device__ __forceinline__ unsigned long long max_with_lane(unsigned long long v) {
  const uint32_t lo = static_cast<uint32_t>(xor_lane_bits<O>(static_cast<int>(static_cast<uint32_t>(v))));
  const uint32_t hi = static_cast<uint32_t>(xor_lane_bits<O>(static_cast<int>(static_cast<uint32_t>(v >> 32))));
  return umax64(v, (static_cast<unsigned long long>(hi) << 32) | lo);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v) {
  v = max_with_lane<32>(v);
  v = max_with_lane<16>(v);
  v = max_with_lane<8>(v);
  v = max_with_lane<4>(v);
  v = max_with_lane<2>(v);
  return max_with_lane<1>(v);
}

// Maximum key over a block (any size that is a multiple of 64, at most 1024).
// Every thread gets the result. `lds` holds 16 entries.
__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v,
                                                            unsigned long long* lds) {
  v = wave_max_u64(v);
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int waves = static_cast<int>(blockDim.x) >> 6;
  if (lane_id() == 0) lds[wave] = v;
  __syncthreads();
  unsigned long long best = 0;
  for (int w = 0; w < waves; ++w) best = umax64(best, lds[w]);
  __syncthreads();
  return best;
}

__device__ __forceinline__ int32_t argmax_id(unsigned long long key) {
  return static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull));
}

// Device state of a sampled generation loop: the draws, the draw counter, and
// where the id goes besides the output (see sample_kernel). All null for a
// plain call.
struct SampleStepState {
  const float* uniforms = nullptr;   // [steps] draws
  int32_t* counter = nullptr;        // [1] index of this step's draw
  int draws = 0;                     // entries of `uniforms`; the index is clamped to them
  int32_t* next_token = nullptr;     // [1] the next step's input
  int32_t* history = nullptr;        // [history_len] history[position + 1] = id
  int history_len = 0;
  int32_t* position = nullptr;       // [1] advanced by one
  uint32_t* epoch = nullptr;         // [1] advanced by one (the decode step's step counter)
};

// Steps 2-6 of the stochastic path after an output head that wrote its
// blocks' argmax keys to `block_best` (the fused decode step's lm_head); the
// scratch is laid out as lcr_sample's (lcr_sample_scratch_floats).
void enqueue_sample_step(const float* logits, int vocab, float temperature, int top_k, float top_p,
                         const unsigned long long* block_best, int best_blocks, float* scratch,
                         int32_t* out_id, const SampleStepState& step, hipStream_t stream);

}  // namespace lcr
