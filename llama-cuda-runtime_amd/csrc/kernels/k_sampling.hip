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


// Inclusive prefix sum over the 64 lanes of a wave (integers: exact in any
// order), on DPP: within each row of 16 lanes by shifts of 1, 2, 4 and 8
// (lanes shifted in from outside the row read 0), then the total of row 0
// into row 1 and of row 2 into row 3 (row_bcast:15), then that of rows 0-1
// into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ int wave_inclusive_scan_int(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15, rows 1 and 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31, rows 2 and 3
  return v;
}

__device__ __forceinline__ int wave_sum_int(int v) {
  v += xor_lane_bits<32>(v);
  v += xor_lane_bits<16>(v);
  v += xor_lane_bits<8>(v);
  v += xor_lane_bits<4>(v);
  v += xor_lane_bits<2>(v);
  return v + xor_lane_bits<1>(v);
}

// The maximum logit from the argmax blocks' partial keys (exact in any
// order): the value half of the largest key. Every lane of the wave gets it.
// The first 256 keys are all requested before any is compared (a loop would
// wait for each load before issuing the next); indices past the last key
// read the last key again, which leaves the maximum unchanged and keeps the
// loads unconditional (blocks >= 1).
__device__ __forceinline__ float max_from_keys(const unsigned long long* __restrict__ block_best, int blocks) {
  constexpr int kAtOnce = 4;
  const int lane = lane_id();
  unsigned long long first[kAtOnce];
#pragma unroll
  for (int j = 0; j < kAtOnce; ++j) first[j] = block_best[min(lane + 64 * j, blocks - 1)];
  unsigned long long key = umax64(umax64(first[0], first[1]), umax64(first[2], first[3]));
  for (int b = lane + 64 * kAtOnce; b < blocks; b += 64) key = umax64(key, block_best[b]);
  key = wave_max_u64(key);
  const uint32_t k = static_cast<uint32_t>(key >> 32);
  return u32_as_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Step 2 over many compute units: block b runs threads 64 b .. 64 b + 63
// of the 1024-thread order, each adding exp(scaled_i) for i = t, t + 1024,
// ... in order, exactly as one 1024-thread block would; the thread's partial
// sum goes to partial_sums[t] and the block's histogram of bins to
// block_hist[b][bin] (counts, so their order of addition is free). The
// block's 16 waves share its 64 chains: wave w computes the exponentials of
// terms w, w + 16, ..., w + 112 of a batch of 128 for every chain (lane l,
// chain 64 b + l: each load reads 64 consecutive logits), all of its loads in
// flight at once, and stages them in LDS by term; then wave 0's lane l adds
// chain l's terms in term order, so the sum is the chain's, bit for bit. One
// batch covers vocabularies up to 131072 entries.
constexpr int kSumChains = 64;                           // chains per block
constexpr int kSumBlocks = kSampleThreads / kSumChains;
constexpr int kSumWaves = 16;
constexpr int kSumTerms = 8;                             // terms per lane per batch
constexpr int kSumBatch = kSumWaves * kSumTerms;         // terms per chain per batch
constexpr int kSumThreads = 64 * kSumWaves;

__global__ __launch_bounds__(kSumThreads) void sample_sum_kernel(float* __restrict__ partial_sums,
                                                                 int* __restrict__ block_hist,
                                                                 const unsigned long long* __restrict__ block_best,
                                                                 int best_blocks, const float* __restrict__ logits,
                                                                 int vocab, float inv_temperature) {
  __shared__ int hist[kHistogramBins];
  __shared__ float stage[kSumBatch][kSumChains];
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int chain = static_cast<int>(blockIdx.x) * kSumChains + lane;
  // Terms of this lane's chain (none for a chain at or past the vocabulary's
  // end); the block's first chain has the most, which bounds the loop
  // uniformly over the block.
  const int chain_terms = chain < vocab ? (vocab - 1 - chain) / kSampleThreads + 1 : 0;
  const int block_chain = static_cast<int>(blockIdx.x) * kSumChains;
  float e[kSumTerms];
  auto load_batch = [&](int first) {
#pragma unroll
    for (int j = 0; j < kSumTerms; ++j) {
      const int k = first + wave + kSumWaves * j;
      e[j] = k < chain_terms ? logits[chain + k * kSampleThreads] : 0.0f;
    }
  };
  // The first batch's logits are requested before the maximum, which they
  // do not depend on, so the two reads overlap.
  load_batch(0);
  const float max_logit = max_from_keys(block_best, best_blocks);
  for (int b = threadIdx.x; b < kHistogramBins; b += kSumThreads) hist[b] = 0;
  __syncthreads();
  float local_sum = 0.0f;
  int last_bin = 0;
  for (int first = 0; block_chain + first * kSampleThreads < vocab; first += kSumBatch) {
    if (first > 0) load_batch(first);
#pragma unroll
    for (int j = 0; j < kSumTerms; ++j) {
      const int k = first + wave + kSumWaves * j;
      const float scaled = (e[j] - max_logit) * inv_temperature;
      stage[wave + kSumWaves * j][lane] = k < chain_terms ? lcr_expf(scaled) : 0.0f;
      if (k < chain_terms) {
        const int bin = min(kHistogramBins - 1, static_cast<int>(-scaled * (kHistogramBins / 20.0f)));
        if (bin == kHistogramBins - 1) {
          ++last_bin;
        } else if (bin >= 0) {
          atomicAdd(&hist[bin], 1);
        }
      }
    }
    __syncthreads();
    if (wave == 0) {
      // Terms past the chain's end are staged as +0, and adding +0 to a sum
      // of exponentials (never -0) leaves its bits unchanged, so every slot
      // is added; reads go 32 at a time ahead of their adds.
#pragma unroll
      for (int k0 = 0; k0 < kSumBatch; k0 += 32) {
        float t[32];
#pragma unroll
        for (int u = 0; u < 32; ++u) t[u] = stage[k0 + u][lane];
#pragma unroll
        for (int u = 0; u < 32; ++u) local_sum += t[u];
      }
    }
    __syncthreads();
  }
  last_bin = wave_sum_int(last_bin);
  if (wave == 0) partial_sums[chain] = local_sum;
  if (lane == 0) atomicAdd(&hist[kHistogramBins - 1], last_bin);
  __syncthreads();
  for (int b = threadIdx.x; b < kHistogramBins; b += kSumThreads) {
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

// What a sampled step reads of the device-resident generation loop's state:
// the draw index (clamped to the draws), its uniform, the position and the
// step counter (for a single call: draw 0, the caller's uniform).
struct StepValues {
  int draw;
  float u;
  int position;
  uint32_t epoch;
};

__device__ __forceinline__ StepValues load_step_values(const SampleStepState& step, float uniform) {
  StepValues sv{0, uniform, 0, 0u};
  if (step.counter != nullptr) {
    sv.position = *step.position;
    if (step.epoch != nullptr) sv.epoch = *step.epoch;
    sv.draw = min(max(*step.counter, 0), step.draws - 1);
    sv.u = step.uniforms[sv.draw];
  }
  return sv;
}

// The sampled id's stores: the output, and in a device-resident generation
// loop the next step's input, the history, the position, the draw counter
// and the step counter.
__device__ __forceinline__ void finish_sample(int32_t* out_id, int picked, const StepValues& sv,
                                              const SampleStepState& step) {
  *out_id = picked;
  if (step.counter != nullptr) {
    *step.next_token = picked;
    if (sv.position + 1 < step.history_len) step.history[sv.position + 1] = picked;
    *step.position = sv.position + 1;
    *step.counter = sv.draw + 1;
    if (step.epoch != nullptr) *step.epoch = sv.epoch + 1u;
  }
}

// The value of lane (lane ^ step), step a power of two below 64 that is a
// constant once the loops around the call are unrolled: DPP and LDS swizzles
// for the short distances (xor_lane), which move the same bits as a general
// shuffle without its address computation and LDS round trip.
template <typename T>
__device__ __forceinline__ T xor_lane_step(T v, int step) {
  static_assert(sizeof(T) == 4, "one 32-bit lane value");
  const float f = __builtin_bit_cast(float, v);
  float r;
  switch (step) {
    case 1: r = xor_lane<1>(f); break;
    case 2: r = xor_lane<2>(f); break;
    case 4: r = xor_lane<4>(f); break;
    case 8: r = xor_lane<8>(f); break;
    case 16: r = xor_lane<16>(f); break;
    default: r = xor_lane<32>(f); break;
  }
  return __builtin_bit_cast(T, r);
}

// A candidate's place in the order (value desc, index asc) as one unsigned
// 64-bit key: the argmax key of sampling.h (order-preserving value bits over
// the complemented index), with -0 taken as +0 so that equal values tie on
// the index alone (both weigh exp(0) = 1). The key round-trips the value and
// the index. Empty places hold 0, below every candidate; NaN values have no
// defined place.
__device__ __forceinline__ unsigned long long cand_key(float v, int idx) {
  return argmax_key(v == 0.0f ? 0.0f : v, static_cast<uint32_t>(idx));
}

__device__ __forceinline__ float key_value(unsigned long long key) {
  const uint32_t k = static_cast<uint32_t>(key >> 32);
  return u32_as_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

__device__ __forceinline__ int key_index(unsigned long long key) {
  return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key));
}

__device__ __forceinline__ unsigned long long xor_lane_key(unsigned long long key, int step) {
  const uint32_t lo = xor_lane_step(static_cast<uint32_t>(key), step);
  const uint32_t hi = xor_lane_step(static_cast<uint32_t>(key >> 32), step);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// One compare-exchange step of the bitonic sort with the key of thread
// t ^ step: thread t keeps the key that ranks first when it is the lower of
// the pair in an ascending run (or the upper in a descending one), else the
// other, which is the swap of the pairwise formulation.
__device__ __forceinline__ void bitonic_keep(unsigned long long& key, unsigned long long partner, int t, int span,
                                             int step) {
  const bool keep_first = ((t & step) == 0) == ((t & span) == 0);
  if (keep_first == (partner > key)) key = partner;
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
  __shared__ unsigned long long keys[kMaxCandidates];
  __shared__ StepValues shared_step;
  const int t = threadIdx.x;
  const int lane = lane_id();
  const int wave = t >> 6;
  static_assert(kSampleThreads == kMaxCandidates, "one candidate per thread");

  const float partial = partial_sums[t];
  // The step state, read by wave 1 (idle until the sum's barriers) so that
  // its dependent reads (the counter, then the uniform it indexes) pass
  // under wave 0's scan; the sum's barriers publish it.
  if (t == 64) shared_step = load_step_values(step, uniform);

  // Where each block's list starts in the merged order (wave 0, exclusive
  // scan over the blocks, 64 at a time). The counts of the first
  // kCountChunks chunks are all requested before the first is scanned.
  if (wave == 0) {
    constexpr int kCountChunks = 4;
    int counts[kCountChunks];
#pragma unroll
    for (int k = 0; k < kCountChunks; ++k) {
      const int b = 64 * k + lane;
      counts[k] = b < compact_blocks ? cand_counts[b] : 0;
    }
    int carry = 0;
    auto scan_chunk = [&](int base, int count) {
      const int b = base + lane;
      const int incl = wave_inclusive_scan_int(count);
      if (b < compact_blocks) block_start[b] = carry + incl - count;
      carry += __builtin_amdgcn_readlane(incl, 63);
    };
#pragma unroll
    for (int k = 0; k < kCountChunks; ++k) {
      if (64 * k < compact_blocks) scan_chunk(64 * k, counts[k]);
    }
    for (int base = 64 * kCountChunks; base < compact_blocks; base += 64) {
      scan_chunk(base, base + lane < compact_blocks ? cand_counts[base + lane] : 0);
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
    // Within block lo_b's list by construction; clamped into the lists all
    // the same, so no start table can send the read elsewhere.
    const int in_list = min(max(t - block_start[lo_b], 0), kCompactSlice - 1);
    const size_t at = static_cast<size_t>(lo_b) * kCompactSlice + static_cast<size_t>(in_list);
    v = cand_values[at];
    idx = cand_indices[at];
  }

  // 5. Order (value desc, index asc), one key per thread.
  unsigned long long key = t < found ? cand_key(v, idx) : 0ull;
  if (top_k > 0 && top_k <= 64) {
    // The walk reads only the first top_k: the best 64 in order suffice. Each
    // wave sorts its 64 (best at lane 0); then four levels merge the waves'
    // lists in pairs, keeping the better 64 of each pair: for two lists in
    // that order the better of A[l] and B[63 - l] is a bitonic sequence
    // holding the pair's best 64, which steps 32 .. 1 of the sort put in
    // order. The order is total (indices are distinct), so these 64 and
    // their order are the full sort's first 64. Wave 0 ends with them.
#pragma unroll
    for (int span = 2; span <= 64; span <<= 1) {
#pragma unroll
      for (int step = span >> 1; step > 0; step >>= 1) {
        bitonic_keep(key, xor_lane_key(key, step), lane, span, step);
      }
    }
    for (int lists = kSampleThreads / 64; lists > 1; lists >>= 1) {
      keys[t] = key;
      __syncthreads();
      if (wave < lists / 2) {
        const unsigned long long other = keys[(wave + lists / 2) * 64 + 63 - lane];
        if (other > key) key = other;
#pragma unroll
        for (int step = 32; step > 0; step >>= 1) {
          bitonic_keep(key, xor_lane_key(key, step), lane, 64, step);
        }
      }
      __syncthreads();
    }
    // Wave 0 holds the best 64 in order, rank r in lane r. The walk's two
    // loops add the same terms in the same order (fma(weight_i, 1 / total,
    // running) from 0), so both read the prefixes of one chain: every lane
    // runs that chain over the 64 ranks and keeps prefix r in lane r, and
    // the cut (the first rank whose prefix reaches top_p, within top_k) and
    // the pick (the first kept rank whose prefix reaches the target) are the
    // lowest set bits of two ballots.
    if (wave == 0) {
      const float weight = t < found ? lcr_expf(key_value(key)) : 0.0f;
      const int limit = min(found, top_k);
      const float inv_total = 1.0f / total_sum;
      float chain = 0.0f, prefix = 0.0f;
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        chain = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(weight), i)), inv_total,
                               chain);
        prefix = lane == i ? chain : prefix;
      }
      const unsigned long long cross = __ballot(lane < limit && top_p < 1.0f && prefix >= top_p);
      const int walked = cross != 0 ? __ffsll(cross) : limit;  // ranks the first loop takes
      const float kept_mass =
          walked > 0 ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prefix), walked - 1)) : 0.0f;
      const int keep = max(walked, 1);
      const StepValues sv = shared_step;
      const float target = sv.u * kept_mass;
      const unsigned long long hit = __ballot(lane < keep && prefix >= target);
      const int rank = hit != 0 ? __ffsll(hit) - 1 : keep - 1;
      const int picked = __builtin_amdgcn_readlane(key_index(key), rank);
      if (t == 0) finish_sample(out_id, picked, sv, step);
    }
    return;
  }
  // Bitonic sort of all candidates.
  for (int span = 2; span <= kMaxCandidates; span <<= 1) {
    for (int step = span >> 1; step > 0; step >>= 1) {
      unsigned long long partner;
      if (step < 64) {
        const uint32_t lo = __shfl_xor(static_cast<uint32_t>(key), step, 64);
        const uint32_t hi = __shfl_xor(static_cast<uint32_t>(key >> 32), step, 64);
        partner = (static_cast<unsigned long long>(hi) << 32) | lo;
      } else {
        keys[t] = key;
        __syncthreads();
        partner = keys[t ^ step];
        __syncthreads();
      }
      bitonic_keep(key, partner, t, span, step);
    }
  }
  v = key_value(key);
  idx = key_index(key);
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
    const StepValues sv = shared_step;
    const float target = sv.u * kept_mass;
    int picked = indices[0];
    float running = 0.0f;
    for (int i = 0; i < keep; ++i) {
      running = __builtin_fmaf(weights[i], inv_total, running);
      picked = indices[i];
      if (running >= target) break;
    }
    finish_sample(out_id, picked, sv, step);
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
  sample_sum_kernel<<<kSumBlocks, kSumThreads, 0, s>>>(sums, hist, best, blocks, logits, vocab, inv_temperature);
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
  sample_sum_kernel<<<kSumBlocks, kSumThreads, 0, s>>>(sums, hist, block_best, best_blocks, logits, vocab,
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
