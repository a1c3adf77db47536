// Rotary position embedding (the reference's src/kernels/rope.cu:33-87).
//
// Llama pairs element i of a head with element i + head_dim/2 (half-split, not
// interleaved). For angle a = float(position) * inv_freq[i] (one fp32 multiply):
//   out[i]        = lo * cos(a) - hi * sin(a)
//   out[i + half] = hi * cos(a) + lo * sin(a)
// computed as separate multiplies and a subtract/add (no fusion), with
// sin/cos from lcr_sincosf. The query kernel writes the head-major
// [num_heads][tokens][head_dim] layout; the key kernel writes K (rotated) and V
// (copied) straight into the cache at KvCacheView::offset.
#include <algorithm>

#include "../capi_util.h"
#include "../kv_cache.h"
#include "device_common.h"

namespace lcr {
namespace {

__device__ __forceinline__ void rotate_pair(float lo, float hi, float position, float freq,
                                            float* out_lo, float* out_hi) {
  float s, c;
  lcr_sincosf(position * freq, &s, &c);
  *out_lo = lo * c - hi * s;
  *out_hi = hi * c + lo * s;
}

__global__ void rope_q_kernel(elem_t* __restrict__ q_heads, const elem_t* __restrict__ q_proj,
                              const float* __restrict__ inv_freq, int tokens, int start_position,
                              int head_dim, int src_row_stride) {
  const int t = blockIdx.x;
  const int h = blockIdx.y;
  const int half = head_dim / 2;
  const float position = static_cast<float>(start_position + t);
  const int64_t src = static_cast<int64_t>(t) * src_row_stride + static_cast<int64_t>(h) * head_dim;
  const int64_t dst = (static_cast<int64_t>(h) * tokens + t) * head_dim;
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    float a, b;
    rotate_pair(elem_to_float(q_proj[src + i]), elem_to_float(q_proj[src + i + half]), position,
                inv_freq[i], &a, &b);
    q_heads[dst + i] = float_to_elem(a);
    q_heads[dst + i + half] = float_to_elem(b);
  }
}

template <bool kPaged>
__global__ void rope_write_kv_kernel(KvCacheView view, const elem_t* __restrict__ k_proj,
                                     const elem_t* __restrict__ v_proj,
                                     const float* __restrict__ inv_freq, int start_position,
                                     int src_row_stride) {
  const int t = blockIdx.x;
  const int h = blockIdx.y;
  const int head_dim = view.head_dim;
  const int half = head_dim / 2;
  const int position = start_position + t;
  const int64_t src = static_cast<int64_t>(t) * src_row_stride + static_cast<int64_t>(h) * head_dim;
  const size_t dst = view.offset<kPaged>(h, position);
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    float a, b;
    rotate_pair(elem_to_float(k_proj[src + i]), elem_to_float(k_proj[src + i + half]),
                static_cast<float>(position), inv_freq[i], &a, &b);
    view.keys[dst + i] = float_to_elem(a);
    view.keys[dst + i + half] = float_to_elem(b);
  }
  for (int i = threadIdx.x; i < head_dim; i += blockDim.x) view.values[dst + i] = v_proj[src + i];
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" int lcr_rope_q(void* q_heads, const void* q_proj, const float* inv_freq, int tokens,
                          int start_position, int num_heads, int head_dim, int src_row_stride,
                          void* stream) {
  CAPI_CHECK(tokens >= 0 && num_heads >= 0, "rope_q needs non-negative sizes");
  if (tokens == 0 || num_heads == 0) return LCR_OK;
  CAPI_CHECK(head_dim > 0 && head_dim % 2 == 0,
             "head_dim must be positive and even for RoPE, got " << head_dim);
  const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(num_heads));
  const int block = std::min(256, ((head_dim / 2 + 63) / 64) * 64);
  rope_q_kernel<<<grid, block, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<elem_t*>(q_heads), static_cast<const elem_t*>(q_proj), inv_freq, tokens,
      start_position, head_dim, src_row_stride);
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_rope_write_kv(const lcr_kv_view* view, const void* k_proj, const void* v_proj,
                                 const float* inv_freq, int tokens, int start_position, int paged,
                                 int src_row_stride, void* stream) {
  CAPI_CHECK(view != nullptr, "rope_write_kv needs a cache view");
  CAPI_CHECK(tokens >= 0, "rope_write_kv needs a non-negative token count");
  if (tokens == 0) return LCR_OK;
  const KvCacheView v = KvCacheView::from_c(*view);
  CAPI_CHECK(v.head_dim > 0 && v.head_dim % 2 == 0,
             "head_dim must be positive and even for RoPE, got " << v.head_dim);
  CAPI_CHECK(!paged || v.page_table != nullptr, "a paged cache view needs a page table");
  const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(v.num_kv_heads));
  const int block = std::min(256, ((v.head_dim + 63) / 64) * 64);
  auto s = static_cast<hipStream_t>(stream);
  auto* k = static_cast<const elem_t*>(k_proj);
  auto* vv = static_cast<const elem_t*>(v_proj);
  if (paged) {
    rope_write_kv_kernel<true><<<grid, block, 0, s>>>(v, k, vv, inv_freq, start_position, src_row_stride);
  } else {
    rope_write_kv_kernel<false><<<grid, block, 0, s>>>(v, k, vv, inv_freq, start_position, src_row_stride);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}
