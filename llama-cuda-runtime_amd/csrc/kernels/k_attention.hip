// Attention launchers of the kernel ABI: split-K decode attention (+ merge),
// the prefill causal softmax and the paged-cache gather.
//
// Dispatch and argument checks follow the reference's
// src/kernels/attention.cu:327-463 (same compiled head_dim {64, 128} and group
// sizes {1, 2, 4, 8}, same messages); the device work is in
// attention_decode.h. The causal softmax keeps the reference's block shape
// (src/kernels/attention.cu:42-100): 256 threads per (row, head), an online
// (max, sum) per thread over keys t, t+256, ..., a butterfly of
// softmax_combine inside each 32-thread group (offsets 16..1, thread i
// combining its own state with thread i^o's, in that argument order), then the
// 8 group results combined in order by thread 0.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "../capi_util.h"
#include "attention_decode.h"

namespace lcr {
namespace {

// One block per (query head, split); query head h reads kv head h / kGroup.
template <bool kPaged, int kHeadDim, int kGroup>
__global__ __launch_bounds__(kAttnThreads) void decode_attention_kernel(
    elem_t* __restrict__ out, float* __restrict__ partials, const elem_t* __restrict__ q,
    KvCacheView view, int seq_len, float scale, int splits) {
  __shared__ AttnShared<kPaged, kHeadDim, 1> sh;
  decode_attention_block<kPaged, kHeadDim, 1>(sh, out, partials, q, view, blockIdx.x / kGroup,
                                           blockIdx.x, blockIdx.y, splits, seq_len, scale);
}

__global__ __launch_bounds__(kMergeThreads) void merge_splits_kernel(elem_t* __restrict__ out,
                                                                   const float* __restrict__ partials,
                                                                   int splits, int head_dim) {
  __shared__ float lds[kMergeLdsFloats];
  merge_split_partials(out, partials, blockIdx.x, splits, head_dim, lds);
}

constexpr int kSoftmaxThreads = 256;

__global__ __launch_bounds__(kSoftmaxThreads) void causal_softmax_kernel(
    elem_t* __restrict__ probs, const float* __restrict__ scores, int rows, int keys,
    int start_position) {
  __shared__ float group_m[kSoftmaxThreads / 32];
  __shared__ float group_l[kSoftmaxThreads / 32];
  __shared__ float row_stats[2];
  const int row = blockIdx.x;
  const int head = blockIdx.y;
  const int t = threadIdx.x;
  const int64_t base = (static_cast<int64_t>(head) * rows + row) * keys;
  const int limit = min(keys, start_position + row + 1);

  float m = kSoftmaxIdentity;
  float l = 0.0f;
  // Keys t, t + 256, ... in that order, four loads in flight at a time.
  constexpr int kBatch = 4;
  for (int k0 = t; k0 < limit; k0 += kBatch * kSoftmaxThreads) {
    float s[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int k = k0 + b * kSoftmaxThreads;
      s[b] = k < limit ? scores[base + k] : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      if (k0 + b * kSoftmaxThreads < limit) {
        const float merged = fmaxf(m, s[b]);
        l = __builtin_fmaf(l, lcr_expf(m - merged), lcr_expf(s[b] - merged));
        m = merged;
      }
    }
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    const float om = __shfl_xor(m, o, 64);
    const float ol = __shfl_xor(l, o, 64);
    softmax_combine(&m, &l, om, ol);
  }
  if ((t & 31) == 0) {
    group_m[t >> 5] = m;
    group_l[t >> 5] = l;
  }
  __syncthreads();
  if (t == 0) {
    float tm = group_m[0];
    float tl = group_l[0];
    for (int w = 1; w < kSoftmaxThreads / 32; ++w) softmax_combine(&tm, &tl, group_m[w], group_l[w]);
    row_stats[0] = tm;
    row_stats[1] = tl;
  }
  __syncthreads();
  const float row_max = row_stats[0];
  const float inv = 1.0f / row_stats[1];
  for (int k0 = t; k0 < keys; k0 += kBatch * kSoftmaxThreads) {
    float s[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int k = k0 + b * kSoftmaxThreads;
      s[b] = k < limit ? scores[base + k] : 0.0f;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int k = k0 + b * kSoftmaxThreads;
      if (k < keys) probs[base + k] = float_to_elem(k < limit ? lcr_expf(s[b] - row_max) * inv : 0.0f);
    }
  }
}

__global__ void gather_kv_kernel(elem_t* __restrict__ out_keys, elem_t* __restrict__ out_values,
                                 KvCacheView view, int positions) {
  const int position = blockIdx.x;
  const int head = blockIdx.y;
  const size_t src = view.offset<true>(head, position);
  const size_t dst = (static_cast<size_t>(head) * positions + position) * view.head_dim;
  for (int i = threadIdx.x; i < view.head_dim; i += blockDim.x) {
    out_keys[dst + i] = view.keys[src + i];
    out_values[dst + i] = view.values[src + i];
  }
}

struct DecodeArgs {
  elem_t* out;
  float* partials;
  const elem_t* q;
  KvCacheView view;
  int num_heads;
  int seq_len;
  float scale;
  int splits;
  hipStream_t stream;
};

template <bool kPaged, int kHeadDim, int kGroup>
int launch_decode(const DecodeArgs& a) {
  const dim3 grid(static_cast<unsigned>(a.num_heads), static_cast<unsigned>(a.splits));
  decode_attention_kernel<kPaged, kHeadDim, kGroup><<<grid, kAttnThreads, 0, a.stream>>>(
      a.out, a.partials, a.q, a.view, a.seq_len, a.scale, a.splits);
  CAPI_LAUNCHED();
  if (a.splits > 1) {
    merge_splits_kernel<<<a.num_heads, kMergeThreads, 0, a.stream>>>(a.out, a.partials, a.splits, kHeadDim);
    CAPI_LAUNCHED();
  }
  return LCR_OK;
}

template <bool kPaged, int kHeadDim>
int launch_by_group(int heads_per_kv, const DecodeArgs& a) {
  switch (heads_per_kv) {
    case 1: return launch_decode<kPaged, kHeadDim, 1>(a);
    case 2: return launch_decode<kPaged, kHeadDim, 2>(a);
    case 4: return launch_decode<kPaged, kHeadDim, 4>(a);
    case 8: return launch_decode<kPaged, kHeadDim, 8>(a);
    default:
      CAPI_CHECK(false, "decode attention is compiled for 1, 2, 4, or 8 query heads per "
                        "key/value head, this model has " << heads_per_kv);
  }
}

template <bool kPaged>
int launch_by_head_dim(int head_dim, int heads_per_kv, const DecodeArgs& a) {
  switch (head_dim) {
    case 64: return launch_by_group<kPaged, 64>(heads_per_kv, a);
    case 128: return launch_by_group<kPaged, 128>(heads_per_kv, a);
    default:
      CAPI_CHECK(false, "decode attention is compiled for head_dim 64 or 128, this model has "
                            << head_dim);
  }
}

}  // namespace
}  // namespace lcr

// Split partials of lcr_decode_attention_noalloc: one array per device, alive
// until the process ends. Every call on a device shares its array.
static __device__ __align__(256) float scratch[LCR_NOALLOC_ATTENTION_SCRATCH_FLOATS];

namespace lcr {
namespace {

// Device address of `scratch` per device, looked up once (with that device
// current) on the entry point's first call there. In host code the array's
// name is only a host-side stand-in, never a device address.
constexpr int kMaxDevices = 64;
std::atomic<float*> g_noalloc_scratch[kMaxDevices];
std::mutex g_noalloc_mutex;

int noalloc_scratch(float** out) {
  int device = -1;
  CAPI_HIP(hipGetDevice(&device));
  CAPI_CHECK(device >= 0 && device < kMaxDevices,
             "device " << device << " is beyond the " << kMaxDevices << " this library tracks");
  float* ptr = g_noalloc_scratch[device].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_noalloc_mutex);
    ptr = g_noalloc_scratch[device].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      void* address = nullptr;
      CAPI_HIP(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)));
      CAPI_CHECK(address != nullptr, "hipGetSymbolAddress gave no address for the attention scratch");
      ptr = static_cast<float*>(address);
      g_noalloc_scratch[device].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return LCR_OK;
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" size_t lcr_decode_attention_scratch_floats(int num_heads, int head_dim, int splits) {
  if (splits <= 1) return 0;
  return static_cast<size_t>(num_heads) * static_cast<size_t>(splits) *
         static_cast<size_t>(kPartialHeader + head_dim);
}

// Two blocks per compute unit, at least 256 positions per split, 1..64 splits:
// the reference's heuristic (src/kernels/attention.cu:419-431).
extern "C" int lcr_choose_attention_splits(int num_kv_heads, int seq_len, int multiprocessors) {
  const int wanted = std::max(1, 2 * multiprocessors);
  const int kv = std::max(1, num_kv_heads);
  int splits = (wanted + kv - 1) / kv;
  const int useful = std::max(1, seq_len / 256);
  splits = std::min(splits, useful);
  return std::max(1, std::min(splits, 64));
}

extern "C" int lcr_decode_attention(void* out, const void* q, const lcr_kv_view* view,
                                    int num_heads, int heads_per_kv, int seq_len, float scale,
                                    int paged, int splits, float* partials, void* stream) {
  CAPI_CHECK(view != nullptr, "decode attention needs a cache view");
  CAPI_CHECK(seq_len > 0, "decode attention needs at least one cached position");
  CAPI_CHECK(splits >= 1, "split count must be positive, got " << splits);
  CAPI_CHECK(splits == 1 || partials != nullptr,
             "a split decode attention needs scratch space for the partials");
  CAPI_CHECK(view->head_dim % 32 == 0,
             "decode attention needs head_dim to be a multiple of the warp width, got "
                 << view->head_dim);
  CAPI_CHECK(heads_per_kv > 0 && num_heads % heads_per_kv == 0 &&
                 num_heads / heads_per_kv == view->num_kv_heads,
             "num_heads (" << num_heads << ") must equal num_kv_heads (" << view->num_kv_heads
                           << ") times heads_per_kv (" << heads_per_kv << ")");
  CAPI_CHECK(!paged || view->page_table != nullptr, "a paged cache view needs a page table");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(q) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(view->keys) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(view->values) & 15u) == 0,
             "decode attention needs 16-byte aligned q and cache pointers");
  DecodeArgs a;
  a.out = static_cast<elem_t*>(out);
  a.partials = partials;
  a.q = static_cast<const elem_t*>(q);
  a.view = KvCacheView::from_c(*view);
  a.num_heads = num_heads;
  a.seq_len = seq_len;
  a.scale = scale;
  a.splits = std::min(std::min(splits, seq_len), kMaxSplits);
  a.stream = static_cast<hipStream_t>(stream);
  return paged ? launch_by_head_dim<true>(view->head_dim, heads_per_kv, a)
               : launch_by_head_dim<false>(view->head_dim, heads_per_kv, a);
}

extern "C" int lcr_decode_attention_noalloc(void* out, const void* q, const lcr_kv_view* view,
                                            int num_heads, int heads_per_kv, int seq_len, float scale,
                                            int paged, int splits, void* stream) {
  CAPI_CHECK(view != nullptr, "decode attention needs a cache view");
  CAPI_CHECK(seq_len > 0, "decode attention needs at least one cached position");
  CAPI_CHECK(splits >= 1, "split count must be positive, got " << splits);
  CAPI_CHECK(num_heads > 0 && view->head_dim > 0, "decode attention needs positive head counts and head_dim");
  // The split count the launch will use (lcr_decode_attention clamps the same way).
  const int used_splits = std::min(std::min(splits, seq_len), kMaxSplits);
  const size_t need = lcr_decode_attention_scratch_floats(num_heads, view->head_dim, used_splits);
  CAPI_CHECK(need <= LCR_NOALLOC_ATTENTION_SCRATCH_FLOATS,
             "decode attention without allocation holds at most " << LCR_NOALLOC_ATTENTION_SCRATCH_FLOATS
                 << " partial floats, this call needs " << need << " (" << num_heads << " heads x "
                 << used_splits << " splits x " << (kPartialHeader + view->head_dim)
                 << "); pass fewer splits or call lcr_decode_attention with a workspace");
  float* partials = nullptr;
  if (need > 0) {
    const int status = noalloc_scratch(&partials);
    if (status != LCR_OK) return status;
  }
  return lcr_decode_attention(out, q, view, num_heads, heads_per_kv, seq_len, scale, paged, used_splits, partials,
                              stream);
}

extern "C" int lcr_causal_softmax(void* probs, const float* scores, int num_heads, int rows,
                                  int keys, int start_position, void* stream) {
  CAPI_CHECK(num_heads >= 0 && rows >= 0 && keys >= 0, "causal softmax needs non-negative sizes");
  if (rows == 0 || num_heads == 0) return LCR_OK;
  const dim3 grid(static_cast<unsigned>(rows), static_cast<unsigned>(num_heads));
  causal_softmax_kernel<<<grid, kSoftmaxThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<elem_t*>(probs), scores, rows, keys, start_position);
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_gather_kv(void* out_keys, void* out_values, const lcr_kv_view* view,
                             int positions, void* stream) {
  CAPI_CHECK(view != nullptr, "gather_kv needs a cache view");
  CAPI_CHECK(positions >= 0, "gather_kv needs a non-negative position count");
  if (positions == 0) return LCR_OK;
  CAPI_CHECK(view->page_table != nullptr, "gather_kv reads a paged cache view");
  const KvCacheView v = KvCacheView::from_c(*view);
  const dim3 grid(static_cast<unsigned>(positions), static_cast<unsigned>(v.num_kv_heads));
  const int block = std::min(256, ((v.head_dim + 63) / 64) * 64);
  gather_kv_kernel<<<grid, block, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<elem_t*>(out_keys), static_cast<elem_t*>(out_values), v, positions);
  CAPI_LAUNCHED();
  return LCR_OK;
}
