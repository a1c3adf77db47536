// lcr_sample: greedy argmax and temperature / top-k / top-p sampling. The
// algorithm and its fixed orders are described in sampling.h.
#include <algorithm>
#include <climits>

#include "../capi_util.h"
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

// Loads per thread in flight in the passes over the logits (element i of a
// batch is base + i * kSampleThreads, so each thread keeps its order).
constexpr int kSampleBatch = 8;
// Loads in flight per thread of the sum blocks (one wave per compute unit).
constexpr int kSumBatch = 32;
constexpr int kSampleWaves = kSampleThreads / 64;

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

// Step 2 over many compute units: block b (one wave) runs threads
// 64 b .. 64 b + 63 of the 1024-thread order, each adding exp(scaled_i) for
// i = t, t + 1024, ... in order, exactly as one 1024-thread block would; the
// thread's partial sum goes to partial_sums[t] and the block's histogram of
// bins to block_hist[b][bin] (counts, so their order of addition is free).
constexpr int kSumBlocks = kSampleThreads / 64;

__global__ __launch_bounds__(64) void sample_sum_kernel(float* __restrict__ partial_sums, int* __restrict__ block_hist,
                                                        const unsigned long long* __restrict__ block_best,
                                                        int best_blocks, const float* __restrict__ logits,
                                                        int vocab, float inv_temperature) {
  __shared__ int hist[kHistogramBins];
  const int lane = lane_id();
  const int t = static_cast<int>(blockIdx.x) * 64 + lane;
  const float max_logit = max_from_keys(block_best, best_blocks);
  for (int b = lane; b < kHistogramBins; b += 64) hist[b] = 0;
  __syncthreads();
  float local_sum = 0.0f;
  int last_bin = 0;
  for (int base = t; base < vocab; base += kSumBatch * kSampleThreads) {
    float v[kSumBatch];
#pragma unroll
    for (int k = 0; k < kSumBatch; ++k) {
      const int i = base + k * kSampleThreads;
      v[k] = i < vocab ? logits[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kSumBatch; ++k) {
      if (base + k * kSampleThreads < vocab) {
        const float scaled = (v[k] - max_logit) * inv_temperature;
        local_sum += lcr_expf(scaled);
        const int bin = min(kHistogramBins - 1, static_cast<int>(-scaled * (kHistogramBins / 20.0f)));
        if (bin == kHistogramBins - 1) {
          ++last_bin;
        } else if (bin >= 0) {
          atomicAdd(&hist[bin], 1);
        }
      }
    }
  }
  last_bin = wave_sum_int(last_bin);
  partial_sums[t] = local_sum;
  __syncthreads();
  if (lane == 0) hist[kHistogramBins - 1] += last_bin;
  __syncthreads();
  for (int b = lane; b < kHistogramBins; b += 64) block_hist[blockIdx.x * kHistogramBins + b] = hist[b];
}

// Steps 1-6 after sample_sum_kernel: the maximum and the total from the
// partials (the total in the 1024-thread tree of block_sum_1024), the
// histogram from the blocks' counts, then the cutoff, the compaction, the
// sort and the walk in one 1024-thread block.
__global__ __launch_bounds__(kSampleThreads) void sample_kernel(int32_t* __restrict__ out_id,
                                                                const float* __restrict__ logits,
                                                                int vocab, float inv_temperature,
                                                                int top_k, float top_p,
                                                                float uniform,
                                                                const unsigned long long* __restrict__ block_best,
                                                                int best_blocks,
                                                                const float* __restrict__ partial_sums,
                                                                const int* __restrict__ block_hist) {
  __shared__ float lds32[32];
  __shared__ int histogram[kHistogramBins];
  __shared__ int wave_counts[kSampleWaves];
  __shared__ int shared_cutoff;
  __shared__ float values[kMaxCandidates];
  __shared__ int indices[kMaxCandidates];
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t >> 6;

  // 1. Maximum logit; 2. the exponential sum and the histogram, from the
  // partials of sample_sum_kernel.
  float max_logit = 0.0f;
  if (wave == 0) {
    max_logit = max_from_keys(block_best, best_blocks);
    if (lane == 0) lds32[0] = max_logit;
  }
  for (int b = t; b < kHistogramBins; b += kSampleThreads) {
    int count = 0;
#pragma unroll
    for (int w = 0; w < kSumBlocks; ++w) count += block_hist[w * kHistogramBins + b];
    histogram[b] = count;
  }
  __syncthreads();
  max_logit = lds32[0];
  __syncthreads();
  const float total_sum = block_sum_1024(partial_sums[t], lds32);

  // 3. Cutoff bin: the number of leading bins whose running count stays
  // <= kMaxCandidates (at least 1). Wave 0, four bins per lane, in bin order.
  if (wave == 0) {
    static_assert(kHistogramBins == 4 * 64, "four bins per lane");
    int c[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) c[k] = histogram[4 * lane + k];
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
    if (lane == 0) shared_cutoff = max(fits, 1);
  }
  __syncthreads();
  const int cutoff_bin = shared_cutoff;

  // 4. Ordered compaction. Wave w owns the index range [w * seg, (w + 1) * seg)
  // and walks it 64 consecutive logits per step (coalesced): it counts its
  // candidates, takes the exclusive prefix over the waves, then writes them
  // in index order (a lane's slot is the candidates of the lanes below it).
  auto is_candidate = [&](float logit, float* scaled_out) {
    const float scaled = (logit - max_logit) * inv_temperature;
    const int bin = min(kHistogramBins - 1, static_cast<int>(-scaled * (kHistogramBins / 20.0f)));
    *scaled_out = scaled;
    return bin < cutoff_bin;
  };
  const int seg = ((vocab + kSampleWaves - 1) / kSampleWaves + 63) / 64 * 64;
  const int lo = min(vocab, wave * seg);
  const int hi = min(vocab, lo + seg);
  int mine = 0;
  for (int base = lo; base < hi; base += 64 * kSampleBatch) {
    float v[kSampleBatch];
#pragma unroll
    for (int k = 0; k < kSampleBatch; ++k) {
      const int i = base + 64 * k + lane;
      v[k] = i < hi ? logits[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kSampleBatch; ++k) {
      float scaled;
      const bool take = base + 64 * k + lane < hi && is_candidate(v[k], &scaled);
      mine += __popcll(__ballot(take));
    }
  }
  if (lane == 0) wave_counts[wave] = mine;
  __syncthreads();
  int total_found = 0;
  int slot = 0;
  for (int w = 0; w < kSampleWaves; ++w) {
    if (w == wave) slot = total_found;
    total_found += wave_counts[w];
  }
  for (int base = lo; base < hi && slot < kMaxCandidates; base += 64 * kSampleBatch) {
    float v[kSampleBatch];
#pragma unroll
    for (int k = 0; k < kSampleBatch; ++k) {
      const int i = base + 64 * k + lane;
      v[k] = i < hi ? logits[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kSampleBatch; ++k) {
      const int i = base + 64 * k + lane;
      float scaled = 0.0f;
      const bool take = i < hi && is_candidate(v[k], &scaled);
      const unsigned long long mask = __ballot(take);
      const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0));
      if (take && slot + below < kMaxCandidates) {
        values[slot + below] = scaled;
        indices[slot + below] = i;
      }
      slot += __popcll(mask);
    }
  }
  const int found = min(total_found, kMaxCandidates);
  __syncthreads();
  for (int i = t; i < kMaxCandidates; i += kSampleThreads) {
    if (i >= found) {
      values[i] = -FLT_MAX;
      indices[i] = INT_MAX;
    }
  }
  __syncthreads();

  // 5. Bitonic sort into (value desc, index asc).
  for (int span = 2; span <= kMaxCandidates; span <<= 1) {
    for (int step = span >> 1; step > 0; step >>= 1) {
      const int partner = t ^ step;
      if (partner > t) {
        const bool first_half = (t & span) == 0;
        const bool partner_first = ranks_before(values[partner], indices[partner], values[t], indices[t]);
        const bool swap = first_half ? partner_first : !partner_first;
        if (swap) {
          const float tv = values[t];
          values[t] = values[partner];
          values[partner] = tv;
          const int ti = indices[t];
          indices[t] = indices[partner];
          indices[partner] = ti;
        }
      }
      __syncthreads();
    }
  }

  // 6. Walk.
  if (t == 0) {
    const int limit = top_k > 0 ? min(found, top_k) : found;
    const float inv_total = 1.0f / total_sum;
    int keep = 0;
    float kept_mass = 0.0f;
    for (int i = 0; i < limit; ++i) {
      kept_mass = __builtin_fmaf(lcr_expf(values[i]), inv_total, kept_mass);
      ++keep;
      if (top_p < 1.0f && kept_mass >= top_p) break;
    }
    if (keep == 0) keep = 1;
    const float target = uniform * kept_mass;
    int picked = indices[0];
    float running = 0.0f;
    for (int i = 0; i < keep; ++i) {
      running = __builtin_fmaf(lcr_expf(values[i]), inv_total, running);
      picked = indices[i];
      if (running >= target) break;
    }
    *out_id = picked;
  }
}

}  // namespace
}  // namespace lcr

using namespace lcr;

// Scratch floats: one 64-bit partial maximum per argmax block, then (for
// sampling) the 1024 partial exponential sums and the sum blocks' histograms.
constexpr size_t kScratchKeys = 2 * static_cast<size_t>(kArgmaxBlocks);
constexpr size_t kScratchSums = kSampleThreads;
constexpr size_t kScratchHist = static_cast<size_t>(kSumBlocks) * kHistogramBins;

extern "C" size_t lcr_sample_scratch_floats(int vocab, int top_k) {
  (void)vocab;
  (void)top_k;
  return kScratchKeys + kScratchSums + kScratchHist;
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
  const int blocks = std::min(kArgmaxBlocks, (vocab + kArgmaxThreads - 1) / kArgmaxThreads);
  const float inv_temperature = 1.0f / temperature;
  argmax_partial_kernel<<<blocks, kArgmaxThreads, 0, s>>>(best, logits, vocab);
  CAPI_LAUNCHED();
  sample_sum_kernel<<<kSumBlocks, 64, 0, s>>>(sums, hist, best, blocks, logits, vocab, inv_temperature);
  CAPI_LAUNCHED();
  sample_kernel<<<1, kSampleThreads, 0, s>>>(out_id, logits, vocab, inv_temperature, top_k, top_p, uniform, best,
                                             blocks, sums, hist);
  CAPI_LAUNCHED();
  return LCR_OK;
}
