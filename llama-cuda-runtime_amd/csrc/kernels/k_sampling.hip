// lcr_sample: greedy argmax and temperature / top-k / top-p sampling. The
// algorithm and its fixed orders are described in sampling.h.
#include <algorithm>
#include <climits>

#include "../capi_util.h"
#include "../hip_utils.h"
#include "sampling.h"

namespace lcr {
namespace {

__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(
    unsigned long long* __restrict__ block_best, const float* __restrict__ logits, int vocab) {
  __shared__ unsigned long long lds[16];
  const int stride = gridDim.x * kArgmaxThreads;
  unsigned long long local = 0;
  for (int i = blockIdx.x * kArgmaxThreads + threadIdx.x; i < vocab; i += stride) {
    local = umax64(local, argmax_key(logits[i], static_cast<uint32_t>(i)));
  }
  local = block_max_u64(local, lds);
  if (threadIdx.x == 0) block_best[blockIdx.x] = local;
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(
    int32_t* __restrict__ out_id, const unsigned long long* __restrict__ block_best, int blocks) {
  __shared__ unsigned long long lds[16];
  unsigned long long local = 0;
  for (int i = threadIdx.x; i < blocks; i += kArgmaxThreads) local = umax64(local, block_best[i]);
  local = block_max_u64(local, lds);
  if (threadIdx.x == 0) *out_id = argmax_id(local);
}

// Sum over the 1024 threads in the reference's block_reduce_sum order.
__device__ __forceinline__ float block_sum_1024(float v, float* lds32) {
  const int t = threadIdx.x;
  v = half_wave_sum(v);
  if ((t & 31) == 0) lds32[t >> 5] = v;
  __syncthreads();
  float total = 0.0f;
  if (t < 32) total = half_wave_sum(lds32[t]);
  __syncthreads();
  if (t == 0) lds32[0] = total;
  __syncthreads();
  total = lds32[0];
  __syncthreads();
  return total;
}

__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}


__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// The maximum logit from the argmax blocks' partial keys (exact in any
// order): the value half of the largest key. Every lane of the wave gets it.
__device__ __forceinline__ float max_from_keys(const unsigned long long* __restrict__ block_best, int blocks) {
  unsigned long long key = 0;
  for (int b = lane_id(); b < blocks; b += 64) key = umax64(key, block_best[b]);
  key = wave_max_u64(key);
  const uint32_t k = static_cast<uint32_t>(key >> 32);
  return u32_as_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Step 2 over many compute units: block b runs threads 64 b .. 64 b + 63
// of the 1024-thread order, each adding exp(scaled_i) for i = t, t + 1024,
// ... in order, exactly as one 1024-thread block would; the thread's partial
// sum goes to partial_sums[t] and the block's histogram of bins to
// block_hist[b][bin] (counts, so their order of addition is free). Four lanes
// share a thread's chain: lane s of a quad computes the exponentials of terms
// s, s + 4, s + 8, ... and the quad's first lane adds all of them in term
// order, each broadcast to it across the quad, so the sum is the chain's, bit
// for bit, with a quarter of the exponentials per lane.
constexpr int kSumBlocks = kSampleThreads / 64;
constexpr int kSumWaves = 4;                 // per block: 64 chains, 4 lanes each
constexpr int kSumTerms = 8;                 // terms per lane per batch (32 per chain)

template <int S>
__device__ __forceinline__ float quad_lane(float v) {
  constexpr int ctrl = S | (S << 2) | (S << 4) | (S << 6);  // quad_perm [S, S, S, S]
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
}

__global__ __launch_bounds__(64 * kSumWaves) void sample_sum_kernel(float* __restrict__ partial_sums,
                                                                    int* __restrict__ block_hist,
                                                                    const unsigned long long* __restrict__ block_best,
                                                                    int best_blocks, const float* __restrict__ logits,
                                                                    int vocab, float inv_temperature) {
  __shared__ int hist[kHistogramBins];
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int sub = lane & 3;
  const int chain = static_cast<int>(blockIdx.x) * 64 + wave * 16 + (lane >> 2);
  const float max_logit = max_from_keys(block_best, best_blocks);
  for (int b = threadIdx.x; b < kHistogramBins; b += 64 * kSumWaves) hist[b] = 0;
  __syncthreads();
  float local_sum = 0.0f;
  int last_bin = 0;
  // Batch q holds terms 4 kSumTerms q .. 4 kSumTerms (q + 1) - 1 of the
  // chain; this lane's are those congruent to `sub` mod 4.
  for (int first = 0; chain + first * kSampleThreads < vocab; first += 4 * kSumTerms) {
    float e[kSumTerms];
#pragma unroll
    for (int j = 0; j < kSumTerms; ++j) {
      const int i = chain + (first + 4 * j + sub) * kSampleThreads;
      e[j] = i < vocab ? logits[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kSumTerms; ++j) {
      const int i = chain + (first + 4 * j + sub) * kSampleThreads;
      const float scaled = (e[j] - max_logit) * inv_temperature;
      e[j] = lcr_expf(scaled);
      if (i < vocab) {
        const int bin = min(kHistogramBins - 1, static_cast<int>(-scaled * (kHistogramBins / 20.0f)));
        if (bin == kHistogramBins - 1) {
          ++last_bin;
        } else if (bin >= 0) {
          atomicAdd(&hist[bin], 1);
        }
      }
    }
    // In term order: term first + 4 j + s is lane s's e[j].
#pragma unroll
    for (int j = 0; j < kSumTerms; ++j) {
      const float t0 = quad_lane<0>(e[j]);
      const float t1 = quad_lane<1>(e[j]);
      const float t2 = quad_lane<2>(e[j]);
      const float t3 = quad_lane<3>(e[j]);
      const int k = first + 4 * j;
      if (chain + k * kSampleThreads < vocab) local_sum += t0;
      if (chain + (k + 1) * kSampleThreads < vocab) local_sum += t1;
      if (chain + (k + 2) * kSampleThreads < vocab) local_sum += t2;
      if (chain + (k + 3) * kSampleThreads < vocab) local_sum += t3;
    }
  }
  last_bin = wave_sum_int(last_bin);
  if (sub == 0) partial_sums[chain] = local_sum;
  __syncthreads();
  if (lane == 0) atomicAdd(&hist[kHistogramBins - 1], last_bin);
  __syncthreads();
  for (int b = threadIdx.x; b < kHistogramBins; b += 64 * kSumWaves) {
    block_hist[blockIdx.x * kHistogramBins + b] = hist[b];
  }
}

// The cutoff bin of step 3 from the summed histogram (wave 0 of a block; the
// result in *cutoff_out): the number of leading bins whose running count
// stays <= kMaxCandidates, at least 1. Four bins per lane, in bin order.
__device__ __forceinline__ void cutoff_from_histogram(const int* __restrict__ block_hist, int* cutoff_out) {
  static_assert(kHistogramBins == 4 * 64, "four bins per lane");
  const int lane = lane_id();
  int c[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    int count = 0;
#pragma unroll
    for (int w = 0; w < kSumBlocks; ++w) count += block_hist[w * kHistogramBins + 4 * lane + k];
    c[k] = count;
  }
  const int mine = c[0] + c[1] + c[2] + c[3];
  int before = mine;  // inclusive scan of the lane totals
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int other = __shfl_up(before, o, 64);
    if (lane >= o) before += other;
  }
  before -= mine;
  int fits = 0;
  int running = before;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    running += c[k];
    fits += running <= kMaxCandidates ? 1 : 0;
  }
  fits = wave_sum_int(fits);
  if (lane == 0) *cutoff_out = max(fits, 1);
}

// Step 4 over many compute units: block b takes logits
// [b * kCompactSlice, (b + 1) * kCompactSlice) and writes its candidates
// (scaled value, index) in increasing index order to its own list, and their
// count. Wave w of the block owns a contiguous quarter of the slice, 64
// consecutive logits per step; a lane's slot is the candidates of the waves
// and lanes before it. The lists in block order are the compaction in index
// order; the final block keeps their first kMaxCandidates.
constexpr int kCompactThreads = 256;
constexpr int kCompactSlice = 1024;
constexpr int kCompactPer = kCompactSlice / kCompactThreads;  // logits per thread
constexpr int kCompactWaves = kCompactThreads / 64;
constexpr int kMaxCompactBlocks = 1024;  // vocabularies up to 1M entries

__global__ __launch_bounds__(kCompactThreads) void sample_compact_kernel(
    float* __restrict__ cand_values, int* __restrict__ cand_indices, int* __restrict__ cand_counts,
    const float* __restrict__ logits, int vocab, float inv_temperature,
    const unsigned long long* __restrict__ block_best, int best_blocks, const int* __restrict__ block_hist) {
  __shared__ int shared_cutoff;
  __shared__ float shared_max;
  __shared__ int wave_counts[kCompactWaves];
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int lo = static_cast<int>(blockIdx.x) * kCompactSlice;
  // The block's logits, requested before the cutoff is known.
  float v[kCompactPer];
#pragma unroll
  for (int k = 0; k < kCompactPer; ++k) {
    const int i = lo + wave * (kCompactSlice / kCompactWaves) + 64 * k + lane;
    v[k] = i < vocab ? logits[i] : 0.0f;
  }
  if (wave == 0) {
    const float m = max_from_keys(block_best, best_blocks);
    if (lane == 0) shared_max = m;
  } else if (wave == 1) {
    cutoff_from_histogram(block_hist, &shared_cutoff);
  }
  __syncthreads();
  const float max_logit = shared_max;
  const int cutoff_bin = shared_cutoff;
  bool take[kCompactPer];
  float scaled[kCompactPer];
  int mine = 0;
#pragma unroll
  for (int k = 0; k < kCompactPer; ++k) {
    const int i = lo + wave * (kCompactSlice / kCompactWaves) + 64 * k + lane;
    scaled[k] = (v[k] - max_logit) * inv_temperature;
    const int bin = min(kHistogramBins - 1, static_cast<int>(-scaled[k] * (kHistogramBins / 20.0f)));
    take[k] = i < vocab && bin < cutoff_bin;
    mine += __popcll(__ballot(take[k]));
  }
  if (lane == 0) wave_counts[wave] = mine;
  __syncthreads();
  int slot = 0;
  int total = 0;
  for (int w = 0; w < kCompactWaves; ++w) {
    if (w == wave) slot = total;
    total += wave_counts[w];
  }
  float* values = cand_values + static_cast<size_t>(blockIdx.x) * kCompactSlice;
  int* indices = cand_indices + static_cast<size_t>(blockIdx.x) * kCompactSlice;
#pragma unroll
  for (int k = 0; k < kCompactPer; ++k) {
    const int i = lo + wave * (kCompactSlice / kCompactWaves) + 64 * k + lane;
    const unsigned long long mask = __ballot(take[k]);
    const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
    if (take[k]) {
      values[slot + below] = scaled[k];
      indices[slot + below] = i;
    }
    slot += __popcll(mask);
  }
  if (threadIdx.x == 0) cand_counts[blockIdx.x] = total;
}

// The sampled id's stores: the output, and in a device-resident generation
// loop the next step's input, the history, the position, the draw counter
// and the step counter.
__device__ __forceinline__ void finish_sample(int32_t* out_id, int picked, int draw, const SampleStepState& step) {
  *out_id = picked;
  if (step.counter != nullptr) {
    const int pos = *step.position;
    *step.next_token = picked;
    if (pos + 1 < step.history_len) step.history[pos + 1] = picked;
    *step.position = pos + 1;
    *step.counter = draw + 1;
    if (step.epoch != nullptr) *step.epoch = *step.epoch + 1u;
  }
}

// One compare-exchange step of the bitonic sort with the element of thread
// t ^ step: thread t keeps the element that ranks first when it is the lower
// of the pair in an ascending run (or the upper in a descending one), else
// the other, which is the swap of the pairwise formulation.
__device__ __forceinline__ void bitonic_keep(float& v, int& i, float pv, int pi, int t, int span, int step) {
  const bool keep_first = ((t & step) == 0) == ((t & span) == 0);
  const bool partner_first = ranks_before(pv, pi, v, i);
  if (keep_first == partner_first) {
    v = pv;
    i = pi;
  }
}

// Steps 1-2's totals and 4-6 after sample_compact_kernel, in one 1024-thread
// block: the maximum is not needed again (the candidates carry their scaled
// values); the total from the partial sums in the 1024-thread tree of
// block_sum_1024; the first kMaxCandidates candidates gathered from the
// blocks' lists in block order; the sort with one element per thread
// (exchanges between lanes of a wave by shuffles, between waves through LDS;
// for top_k <= 64 only the best 64 are put in order);
// the walk with every exponential computed beforehand, one per thread.
// With `step` set (a device-resident generation loop), the uniform is
// step.uniforms[*step.counter], and the id also becomes the next step's input
// and history[position + 1], and the position and the counter advance (what
// argmax_step_kernel does for greedy steps).
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(int32_t* __restrict__ out_id,
                                                                int top_k, float top_p, float uniform,
                                                                const float* __restrict__ partial_sums,
                                                                const float* __restrict__ cand_values,
                                                                const int* __restrict__ cand_indices,
                                                                const int* __restrict__ cand_counts,
                                                                int compact_blocks, SampleStepState step) {
  __shared__ float lds32[32];
  __shared__ int block_start[kMaxCompactBlocks];
  __shared__ int shared_found;
  __shared__ float values[kMaxCandidates];
  __shared__ int indices[kMaxCandidates];
  __shared__ float weights[kMaxCandidates];
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t >> 6;
  static_assert(kSampleThreads == kMaxCandidates, "one candidate per thread");

  const float partial = partial_sums[t];

  // Where each block's list starts in the merged order (wave 0, exclusive
  // scan over the blocks, 64 at a time).
  if (wave == 0) {
    int carry = 0;
    for (int base = 0; base < compact_blocks; base += 64) {
      const int b = base + lane;
      const int count = b < compact_blocks ? cand_counts[b] : 0;
      int incl = count;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int other = __shfl_up(incl, o, 64);
        if (lane >= o) incl += other;
      }
      if (b < compact_blocks) block_start[b] = carry + incl - count;
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) shared_found = min(carry, kMaxCandidates);
  }
  const float total_sum = block_sum_1024(partial, lds32);  // its barriers publish the scan
  const int found = shared_found;
  // Gather: thread t fetches merged candidate t from the last block whose
  // list starts at or before t (binary search over the starts), so every
  // thread's load is in flight at once.
  float v = -FLT_MAX;
  int idx = INT_MAX;
  if (t < found) {
    int lo_b = 0, hi_b = compact_blocks - 1;
    while (lo_b < hi_b) {
      const int mid = (lo_b + hi_b + 1) >> 1;
      if (block_start[mid] <= t) {
        lo_b = mid;
      } else {
        hi_b = mid - 1;
      }
    }
    const size_t at = static_cast<size_t>(lo_b) * kCompactSlice + static_cast<size_t>(t - block_start[lo_b]);
    v = cand_values[at];
    idx = cand_indices[at];
  }

  // 5. Order (value desc, index asc), one element per thread.
  if (top_k > 0 && top_k <= 64) {
    // The walk reads only the first top_k: the best 64 in order suffice. Each
    // wave sorts its 64 (best at lane 0); then four levels merge the waves'
    // lists in pairs, keeping the better 64 of each pair: for two lists in
    // that order the better of A[l] and B[63 - l] is a bitonic sequence
    // holding the pair's best 64, which steps 32 .. 1 of the sort put in
    // order. The order is total (indices are distinct), so these 64 and
    // their order are the full sort's first 64. Wave 0 ends with them.
    for (int span = 2; span <= 64; span <<= 1) {
      for (int step = span >> 1; step > 0; step >>= 1) {
        bitonic_keep(v, idx, __shfl_xor(v, step, 64), __shfl_xor(idx, step, 64), lane, span, step);
      }
    }
    for (int lists = kSampleThreads / 64; lists > 1; lists >>= 1) {
      values[t] = v;
      indices[t] = idx;
      __syncthreads();
      if (wave < lists / 2) {
        const int other = (wave + lists / 2) * 64 + 63 - lane;
        const float ov = values[other];
        const int oi = indices[other];
        if (ranks_before(ov, oi, v, idx)) {
          v = ov;
          idx = oi;
        }
        for (int step = 32; step > 0; step >>= 1) {
          bitonic_keep(v, idx, __shfl_xor(v, step, 64), __shfl_xor(idx, step, 64), lane, 64, step);
        }
      }
      __syncthreads();
    }
    // Wave 0 holds the best 64 in order, rank r in lane r: it walks them
    // itself, reading rank i's weight and index from lane i (the same fma
    // chain, in the same order, as the LDS walk below).
    if (wave == 0) {
      const float weight = t < found ? lcr_expf(v) : 0.0f;
      const int limit = min(found, top_k);
      const float inv_total = 1.0f / total_sum;
      int keep = 0;
      float kept_mass = 0.0f;
      for (int i = 0; i < limit; ++i) {
        kept_mass = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(weight), i)), inv_total,
                                   kept_mass);
        ++keep;
        if (top_p < 1.0f && kept_mass >= top_p) break;
      }
      if (keep == 0) keep = 1;
      const int draw = step.counter != nullptr ? min(max(*step.counter, 0), step.draws - 1) : 0;
      const float u = step.counter != nullptr ? step.uniforms[draw] : uniform;
      const float target = u * kept_mass;
      int picked = __builtin_amdgcn_readlane(idx, 0);
      float running = 0.0f;
      for (int i = 0; i < keep; ++i) {
        running = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(weight), i)), inv_total,
                                 running);
        picked = __builtin_amdgcn_readlane(idx, i);
        if (running >= target) break;
      }
      if (t == 0) finish_sample(out_id, picked, draw, step);
    }
    return;
  } else {
    // Bitonic sort of all candidates.
    for (int span = 2; span <= kMaxCandidates; span <<= 1) {
      for (int step = span >> 1; step > 0; step >>= 1) {
        float pv;
        int pi;
        if (step < 64) {
          pv = __shfl_xor(v, step, 64);
          pi = __shfl_xor(idx, step, 64);
        } else {
          values[t] = v;
          indices[t] = idx;
          __syncthreads();
          pv = values[t ^ step];
          pi = indices[t ^ step];
          __syncthreads();
        }
        bitonic_keep(v, idx, pv, pi, t, span, step);
      }
    }
  }
  values[t] = v;
  indices[t] = idx;
  // The walk's terms, every one computed once (the same values the walk's
  // loop would compute in turn).
  weights[t] = t < found ? lcr_expf(v) : 0.0f;
  __syncthreads();

  // 6. Walk.
  if (t == 0) {
    const int limit = top_k > 0 ? min(found, top_k) : found;
    const float inv_total = 1.0f / total_sum;
    int keep = 0;
    float kept_mass = 0.0f;
    for (int i = 0; i < limit; ++i) {
      kept_mass = __builtin_fmaf(weights[i], inv_total, kept_mass);
      ++keep;
      if (top_p < 1.0f && kept_mass >= top_p) break;
    }
    if (keep == 0) keep = 1;
    const int draw = step.counter != nullptr ? min(max(*step.counter, 0), step.draws - 1) : 0;
    const float u = step.counter != nullptr ? step.uniforms[draw] : uniform;
    const float target = u * kept_mass;
    int picked = indices[0];
    float running = 0.0f;
    for (int i = 0; i < keep; ++i) {
      running = __builtin_fmaf(weights[i], inv_total, running);
      picked = indices[i];
      if (running >= target) break;
    }
    finish_sample(out_id, picked, draw, step);
  }
}

}  // namespace
}  // namespace lcr

using namespace lcr;

// Scratch floats: one 64-bit partial maximum per argmax block, then (for
// sampling) the 1024 partial exponential sums, the sum blocks' histograms,
// and per compaction block its candidate count and its list of (scaled
// value, index).
constexpr size_t kScratchKeys = 2 * static_cast<size_t>(kArgmaxBlocks);
constexpr size_t kScratchSums = kSampleThreads;
constexpr size_t kScratchHist = static_cast<size_t>(kSumBlocks) * kHistogramBins;

static int compact_blocks_for(int vocab) { return (vocab + kCompactSlice - 1) / kCompactSlice; }

extern "C" size_t lcr_sample_scratch_floats(int vocab, int top_k) {
  (void)top_k;
  const size_t blocks = static_cast<size_t>(compact_blocks_for(std::max(vocab, 1)));
  return kScratchKeys + kScratchSums + kScratchHist + blocks * (1 + 2 * static_cast<size_t>(kCompactSlice));
}

extern "C" int lcr_sample(int32_t* out_id, const float* logits, int vocab, float temperature,
                          int top_k, float top_p, float uniform, float* scratch, void* stream) {
  CAPI_CHECK(vocab > 0, "cannot sample from an empty vocabulary");
  auto s = static_cast<hipStream_t>(stream);
  if (temperature <= 0.0f) {
    CAPI_CHECK(scratch != nullptr, "argmax needs scratch space for its partial maxima");
    CAPI_CHECK((reinterpret_cast<uintptr_t>(scratch) & 7u) == 0,
               "argmax scratch must be 8-byte aligned");
    auto* best = reinterpret_cast<unsigned long long*>(scratch);
    const int blocks = std::min(kArgmaxBlocks, (vocab + kArgmaxThreads - 1) / kArgmaxThreads);
    argmax_partial_kernel<<<blocks, kArgmaxThreads, 0, s>>>(best, logits, vocab);
    CAPI_LAUNCHED();
    argmax_final_kernel<<<1, kArgmaxThreads, 0, s>>>(out_id, best, blocks);
    CAPI_LAUNCHED();
    return LCR_OK;
  }
  CAPI_CHECK(top_p > 0.0f && top_p <= 1.0f, "top_p must be in (0, 1], got " << top_p);
  CAPI_CHECK(scratch != nullptr, "sampling needs scratch space for its partial sums");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(scratch) & 7u) == 0, "sampling scratch must be 8-byte aligned");
  auto* best = reinterpret_cast<unsigned long long*>(scratch);
  float* sums = scratch + kScratchKeys;
  int* hist = reinterpret_cast<int*>(scratch + kScratchKeys + kScratchSums);
  const int compact_blocks = compact_blocks_for(vocab);
  CAPI_CHECK(compact_blocks <= kMaxCompactBlocks,
             "sampling supports vocabularies up to " << kMaxCompactBlocks * kCompactSlice << " entries, got " << vocab);
  int* counts = reinterpret_cast<int*>(scratch + kScratchKeys + kScratchSums + kScratchHist);
  float* cand_values = scratch + kScratchKeys + kScratchSums + kScratchHist + compact_blocks;
  int* cand_indices = reinterpret_cast<int*>(cand_values + static_cast<size_t>(compact_blocks) * kCompactSlice);
  const int blocks = std::min(kArgmaxBlocks, (vocab + kArgmaxThreads - 1) / kArgmaxThreads);
  const float inv_temperature = 1.0f / temperature;
  argmax_partial_kernel<<<blocks, kArgmaxThreads, 0, s>>>(best, logits, vocab);
  CAPI_LAUNCHED();
  sample_sum_kernel<<<kSumBlocks, 64 * kSumWaves, 0, s>>>(sums, hist, best, blocks, logits, vocab, inv_temperature);
  CAPI_LAUNCHED();
  sample_compact_kernel<<<compact_blocks, kCompactThreads, 0, s>>>(cand_values, cand_indices, counts, logits, vocab,
                                                                   inv_temperature, best, blocks, hist);
  CAPI_LAUNCHED();
  sample_kernel<<<1, kSampleThreads, 0, s>>>(out_id, top_k, top_p, uniform, sums, cand_values, cand_indices, counts,
                                             compact_blocks, SampleStepState{});
  CAPI_LAUNCHED();
  return LCR_OK;
}

namespace lcr {

// The stochastic path after an output head that already wrote its blocks'
// argmax keys (the fused step's lm_head): steps 2-6 with the step state.
void enqueue_sample_step(const float* logits, int vocab, float temperature, int top_k, float top_p,
                         const unsigned long long* block_best, int best_blocks, float* scratch,
                         int32_t* out_id, const SampleStepState& step, hipStream_t s) {
  LCR_CHECK(temperature > 0.0f, "a sampled step needs a positive temperature");
  LCR_CHECK(top_p > 0.0f && top_p <= 1.0f, "top_p must be in (0, 1], got " << top_p);
  LCR_CHECK(step.counter != nullptr && step.uniforms != nullptr && step.draws > 0,
            "a sampled step needs its draws on the device");
  const int compact_blocks = compact_blocks_for(vocab);
  LCR_CHECK(compact_blocks <= kMaxCompactBlocks, "vocabulary of " << vocab << " entries is too large to sample");
  float* sums = scratch + kScratchKeys;
  int* hist = reinterpret_cast<int*>(scratch + kScratchKeys + kScratchSums);
  int* counts = reinterpret_cast<int*>(scratch + kScratchKeys + kScratchSums + kScratchHist);
  float* cand_values = scratch + kScratchKeys + kScratchSums + kScratchHist + compact_blocks;
  int* cand_indices = reinterpret_cast<int*>(cand_values + static_cast<size_t>(compact_blocks) * kCompactSlice);
  const float inv_temperature = 1.0f / temperature;
  sample_sum_kernel<<<kSumBlocks, 64 * kSumWaves, 0, s>>>(sums, hist, block_best, best_blocks, logits, vocab,
                                                          inv_temperature);
  HIP_CHECK_LAUNCH();
  sample_compact_kernel<<<compact_blocks, kCompactThreads, 0, s>>>(cand_values, cand_indices, counts, logits, vocab,
                                                                   inv_temperature, block_best, best_blocks, hist);
  HIP_CHECK_LAUNCH();
  sample_kernel<<<1, kSampleThreads, 0, s>>>(out_id, top_k, top_p, 0.0f, sums, cand_values, cand_indices, counts,
                                             compact_blocks, step);
  HIP_CHECK_LAUNCH();
}

}  // namespace lcr
